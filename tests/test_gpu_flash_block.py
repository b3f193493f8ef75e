"""GPU parity of the Flash memory block (models/deepseek/layer.py:46-183) at
d = 512: its grouped low-rank projections against an fp64 restatement of the
reference's projection code (models/deepseek/ops/compiled_tensor_ops.py:12-99),
and ``packed`` (query and commit, with the prologue inside the update's WY
kernel or as its own kernel) against the oracle run on the block's own bf16
projection outputs; ``packed_slots`` must equal ``packed`` bit for bit."""

import types

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import host

from memt_gdn2.block import DeepSeekMemoryBlock

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _config(**kw):
    base = dict(hidden_size=256, num_heads=2, head_dim=512, kv_groups=2, q_rank=64, kv_rank=32, gate_rank=32,
                chunk_tokens=64, norm_eps=1e-6, output_softcap=2.0)
    base.update(kw)
    return types.SimpleNamespace(**base)


def _block(dev, cfg, seed=0, fused=True):
    torch.manual_seed(seed)
    block = DeepSeekMemoryBlock(cfg, device=dev, fused_prologue=fused)
    with torch.no_grad():
        for name, p in block.named_parameters():
            if name.endswith("norm.weight") or name.endswith("group_norm"):
                p.copy_(1 + 0.1 * torch.randn_like(p, dtype=torch.float32))
            elif name in ("decay_scale_log", "decay_bias", "g_down.bias"):
                p.copy_(0.3 * torch.randn_like(p, dtype=torch.float32))
            else:
                p.copy_(torch.randn_like(p, dtype=torch.float32) * p.shape[-1] ** -0.5)
    return block


def _latent_norm64(x, w, eps):
    return x * (1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)) * w


def test_flash_projections_match_fp64(dev):
    print("flash block projections", flush=True)
    cfg = _config()
    block = _block(dev, cfg, seed=1)
    T = 37
    hidden = torch.randn(T, cfg.hidden_size, device=dev).to(torch.bfloat16)
    q, k, v, og, erase, write, decay = (host(t)[0].astype(np.float64) for t in block._project(hidden))
    P = {n: host(p).astype(np.float64) for n, p in block.named_parameters()}
    x = host(hidden).astype(np.float64)
    parts = np.split(x @ P["in_proj.weight"].T, np.cumsum([*block.qkv_rows, *block.gate_rows])[:-1], axis=-1)
    G, R = cfg.kv_groups, cfg.kv_rank

    def expand(lat, up, gain):
        z = _latent_norm64(lat.reshape(T, G, R), gain, cfg.norm_eps)
        return np.einsum("tgr,gwr->tgw", z, up).reshape(T, -1)

    refs = {
        "q": _latent_norm64(parts[0], P["q_norm.weight"], cfg.norm_eps) @ P["q_up.weight"].T,
        "k": expand(parts[1], P["k_group_up"], P["k_group_norm"]),
        "v": expand(parts[2], P["v_group_up"], P["v_group_norm"]),
        "erase": parts[3] @ P["b_up.weight"].T,
        "write": parts[4] @ P["w_up.weight"].T,
        "decay": parts[5] @ P["f_down.weight"].T,
        "output_gate": parts[6] @ P["g_down.weight"].T + P["g_down.bias"],
    }
    got = dict(q=q, k=k, v=v, output_gate=og, erase=erase, write=write, decay=decay)
    for name, ref in refs.items():
        # bf16 projections of bf16 intermediates: a few bf16 ulps of the largest value
        assert np.max(np.abs(got[name] - ref)) <= 2e-2 * np.max(np.abs(ref)), name


def _oracle_packed(block, hidden, read_states, lengths, commit, write_states):
    """The reference's packed() order on the oracle, from the block's bf16
    projection outputs."""
    T, H, D = len(hidden), block.num_heads, block.head_dim
    q, k, v, og, erase, write, decay = (host(t)[0] for t in block._project(hidden))
    q, k, v = (x.reshape(1, T, H, D) for x in (q, k, v))
    gate = og.reshape(T * H, D)
    wn = host(block.o_norm.weight)
    rs = host(read_states)
    scale = D ** -0.5
    q_hat = O.l2norm(q, 1e-6, out_bf16=True)[0]
    if not commit:
        read = O.snapshot_read(q_hat, rs, lengths, scale)
        return O.rms_norm_gated(read.reshape(T * H, D), gate, wn, eps=1e-6, softcap=2.0).reshape(T, H * D), None
    g = O.log_decay(decay, host(block.decay_bias), host(block.decay_scale_log), H).reshape(1, T, H, D)
    sb, beta = O.write_gates(erase, write, bf16=True)
    k_til = O.bf16_round(sb.reshape(1, T, H, D) * O.l2norm(k, 1e-6, out_bf16=True)[0])
    read, final = O.token_memory_packed(q_hat, k_til, v, g, beta.reshape(1, T, H, D), rs, host(write_states),
                                        erase=None, lengths=lengths, scale=scale, chunk_tokens=block.chunk_tokens)
    out = O.rms_norm_gated(read.reshape(T * H, D), gate, wn, eps=1e-6, softcap=2.0)
    return out.reshape(T, H * D), final


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("commit", [False, True])
def test_flash_block_packed(dev, commit, fused):
    print(f"flash block packed commit={commit} fused={fused}", flush=True)
    cfg = _config()
    block = _block(dev, cfg, seed=2, fused=fused)
    lengths = [70, 1, 90]
    T = sum(lengths)
    g = torch.Generator(device=dev).manual_seed(5)
    hidden = torch.randn(T, cfg.hidden_size, generator=g, device=dev).to(torch.bfloat16)
    rs = torch.randn(3, 2, 512, 512, generator=g, device=dev) * 0.05
    ws = torch.randn(3, 2, 512, 512, generator=g, device=dev) * 0.05
    out, final = block.packed(hidden, rs, lengths=lengths, commit=commit, write_states=ws)
    out_ref, final_ref = _oracle_packed(block, hidden, rs, lengths, commit, ws)
    assert out.shape == (T, 1024) and out.dtype == torch.bfloat16
    assert O.parity_err(host(out), out_ref, out_bf16=True) <= TOL
    if commit:
        assert O.max_rel_err(host(final), final_ref) <= TOL
    else:
        assert final is None


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("commit", [False, True])
def test_flash_block_slots_match_packed(dev, commit, fused):
    print(f"flash block slots commit={commit} fused={fused}", flush=True)
    cfg = _config()
    block = _block(dev, cfg, seed=3, fused=fused)
    lengths = [40, 100]
    T = sum(lengths)
    g = torch.Generator(device=dev).manual_seed(6)
    hidden = torch.randn(T, cfg.hidden_size, generator=g, device=dev).to(torch.bfloat16)
    pool = torch.randn(4, 1, 2, 512, 512, generator=g, device=dev) * 0.05
    slots = [3, 1]
    before = pool.clone()
    out_ref, final_ref = block.packed(hidden, before[slots, 0], lengths=lengths, commit=commit,
                                      write_states=before[slots, 0])
    out = block.packed_slots(hidden, pool, slots, slots, lengths=lengths, commit=commit)
    torch.cuda.synchronize()
    assert torch.equal(out, out_ref)
    if commit:
        assert torch.equal(pool[slots, 0], final_ref)
    else:
        assert torch.equal(pool, before)
    assert torch.equal(pool[[0, 2]], before[[0, 2]])


def test_flash_block_through_the_runtime(dev):
    """The serving caller with the Flash block: the gather path and the slot
    path give the same residual rows and slot states."""
    from memt_gdn2.runtime import MemoryRequest, MemoryRuntime, plan_of

    print("flash block through the runtime", flush=True)
    cfg = _config()
    block = _block(dev, cfg, seed=4)
    g = torch.Generator(device=dev).manual_seed(8)
    storage0 = torch.randn(5, 1, 2, 512, 512, generator=g, device=dev) * 0.05
    plan = plan_of([(MemoryRequest("c1", "a", "commit"), 50), (MemoryRequest("q1", "b", "query"), 2),
                    (MemoryRequest("c2", "d", "commit"), 70)])
    slot_of = {"c1": 3, "q1": 0, "c2": 4}
    hidden = torch.randn(plan.token_count, cfg.hidden_size, generator=g, device=dev).to(torch.bfloat16)
    results = []
    for slot_io in (False, True):
        pool = types.SimpleNamespace(storage={0: storage0.clone()})
        rt = MemoryRuntime(pool, slot_io=slot_io)
        rt.begin(plan, slot_of=slot_of, memory_read={"a": True, "b": True, "d": True})
        out = torch.empty(plan.token_count, block.value_dim, dtype=hidden.dtype, device=dev)  # [T, H*D] residual
        rt.run_layer(0, hidden, out, block)
        rt.finish(True)
        torch.cuda.synchronize()
        results.append((out, pool.storage[0]))
    assert torch.equal(results[0][0], results[1][0])
    assert torch.equal(results[0][1], results[1][1])
    assert not torch.equal(results[1][1][3], storage0[3])  # the commits wrote their slots
    assert torch.equal(results[1][1][:3], storage0[:3])
