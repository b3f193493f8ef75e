"""GPU parity of the gate/q/k prologue kernel, of the memory block's
``packed`` entry built on it, and of the serving caller over GPU state slots.

The prologue is compared with the oracle's gates and l2norm (fp64, rounded
to bf16 where the reference stores bf16).  fp32 transcendentals may differ
from the fp64 values in their last bits, which can move a bf16 result across
a rounding boundary: the bf16 outputs are allowed one bf16 ulp and must match
exactly almost everywhere."""

import types

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import host

import memt_gdn2
from memt_gdn2.block import QwenMemoryBlock
from memt_gdn2.runtime import MemoryRequest, MemoryRuntime, plan_of

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _bf16_close(x, ref, *, exact_frac=0.99):
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    diff = np.abs(x - ref)
    assert np.all(diff <= O.bf16_ulp(ref) * 1.0001 + 1e-30), float(np.max(diff / (O.bf16_ulp(ref) + 1e-30)))
    assert np.mean(diff == 0) >= exact_frac, float(np.mean(diff == 0))


def _fused_rows(T, H, D, dev, seed):
    """q, k, erase, write as column slices of fused projection outputs (row
    stride > H*D), as the block's split views are; decay contiguous."""
    g = torch.Generator().manual_seed(seed)
    W = H * D
    qkv = (torch.randn(T, 3 * W, generator=g) * 2).to(dev, torch.bfloat16)
    gates = (torch.randn(T, 2 * W + D, generator=g) * 3).to(dev, torch.bfloat16)
    decay = (torch.randn(T, W, generator=g) * 2).to(dev, torch.bfloat16)
    bias = (torch.randn(W, generator=g) * 0.5).to(dev, torch.bfloat16)
    rate = (torch.randn(H, generator=g) * 0.5).to(dev, torch.bfloat16)
    return qkv[:, :W], qkv[:, W:2 * W], decay, bias, rate, gates[:, :W], gates[:, W:2 * W]


def _ref_gates(decay, bias, rate, erase, write, H):
    f, b, s, e, w = (host(x).astype(np.float64) for x in (decay, bias, rate, erase, write))
    g = O.log_decay(f, b, s, H)
    sb, beta = O.write_gates(e, w, bf16=True)
    return g, sb, beta


@pytest.mark.parametrize("T,H,D", [(37, 4, 128), (64, 2, 64), (9, 2, 256), (1, 16, 128), (11, 2, 512)])
def test_write_gates(dev, T, H, D):
    print(f"write_gates T={T} H={H} D={D}", flush=True)
    _, _, decay, bias, rate, erase, write = _fused_rows(T, H, D, dev, seed=T + D)
    sb, beta, g = memt_gdn2.write_gates(decay, bias, rate, erase, write, H)
    g_ref, sb_ref, beta_ref = _ref_gates(decay, bias, rate, erase, write, H)
    gh = host(g).reshape(T, H, D)
    assert np.allclose(gh, g_ref.reshape(T, H, D), rtol=3e-6, atol=1e-30)
    _bf16_close(host(sb).reshape(T, -1), sb_ref)
    _bf16_close(host(beta).reshape(T, -1), beta_ref)


@pytest.mark.parametrize("T,H,D", [(100, 4, 128), (33, 2, 64), (17, 2, 256), (13, 2, 512)])
def test_memory_prologue(dev, T, H, D):
    print(f"memory_prologue T={T} H={H} D={D}", flush=True)
    q, k, decay, bias, rate, erase, write = _fused_rows(T, H, D, dev, seed=7 * T + D)
    assert q.stride(0) == 3 * H * D  # read in place, not copied
    q_hat, k_til, beta, g = memt_gdn2.memory_prologue(q, k, decay, bias, rate, erase, write, H)
    g_ref, sb_ref, beta_ref = _ref_gates(decay, bias, rate, erase, write, H)
    qh = host(q).reshape(T, H, D)
    kh = host(k).reshape(T, H, D)
    q_ref = O.l2norm(qh, 1e-6, out_bf16=True)[0]
    k_ref = O.bf16_round(sb_ref.reshape(T, H, D) * O.l2norm(kh, 1e-6, out_bf16=True)[0])
    assert np.allclose(host(g).reshape(T, H, D), g_ref.reshape(T, H, D), rtol=3e-6, atol=1e-30)
    _bf16_close(host(beta).reshape(T, -1), beta_ref)
    _bf16_close(host(q_hat).reshape(T, H, D), q_ref)
    _bf16_close(host(k_til).reshape(T, H, D), k_ref, exact_frac=0.98)


def test_prologue_rejects_bad_rows(dev):
    q, k, decay, bias, rate, erase, write = _fused_rows(8, 2, 128, dev, seed=1)
    with pytest.raises(ValueError):
        memt_gdn2.write_gates(decay, bias[:-1], rate, erase, write, 2)
    with pytest.raises(ValueError):
        memt_gdn2.write_gates(decay.float(), bias, rate, erase, write, 2)
    with pytest.raises(ValueError):
        memt_gdn2.memory_prologue(q[:4], k, decay, bias, rate, erase, write, 2)
    with pytest.raises(ValueError):  # D = 96 has no compiled variant
        dd = torch.zeros(8, 192, dtype=torch.bfloat16, device=dev)
        memt_gdn2.write_gates(dd, torch.zeros(192, device=dev), torch.zeros(2, device=dev), dd, dd, 2)


def _config(H=2, D=128, hidden=256, chunk_tokens=128):
    return types.SimpleNamespace(hidden_size=hidden, num_heads=H, head_dim=D, chunk_tokens=chunk_tokens,
                                 rms_norm_eps=1e-6, output_gate_softcap=2.0)


def _block(dev, cfg, seed=0):
    torch.manual_seed(seed)
    block = QwenMemoryBlock(cfg, device=dev)
    with torch.no_grad():
        for name, p in block.named_parameters():
            if name.endswith("weight") and p.ndim == 2:
                p.copy_(torch.randn_like(p, dtype=torch.float32) * p.shape[1] ** -0.5)
            elif name == "o_norm.weight":
                p.copy_(1 + 0.1 * torch.randn_like(p, dtype=torch.float32))
            else:
                p.copy_(torch.randn_like(p, dtype=torch.float32) * 0.5)
    return block


def _oracle_packed(block, hidden, read_states, lengths, commit, write_states):
    """The reference's packed() order on the oracle, from the same bf16
    projection outputs the GPU GEMMs produced."""
    T, H, D = len(hidden), block.num_heads, block.head_dim
    W = H * D
    lin = torch.nn.functional.linear
    hb = hidden.unsqueeze(0)
    wt = block.in_proj.weight
    with torch.no_grad():  # the same GEMM calls as the block makes
        qkv = host(lin(hb, wt[:3 * W]))[0]
        gate_out = block.g_down(lin(hb, wt[-D:]))
        gates_t = lin(hb, wt[3 * W:5 * W + D])
        decay = block.f_down(gates_t[..., 2 * W:])
    gates = host(gates_t)[0]
    q, k, v = (qkv[:, i * W:(i + 1) * W].reshape(1, T, H, D) for i in range(3))
    gate = host(gate_out)[0].reshape(T * H, D)
    wn = host(block.o_norm.weight)
    rs = host(read_states)
    scale = D ** -0.5
    q_hat = O.l2norm(q, 1e-6, out_bf16=True)[0]
    if not commit:
        read = O.snapshot_read(q_hat, rs, lengths, scale)
        out = O.rms_norm_gated(read.reshape(T * H, D), gate, wn, eps=1e-6, softcap=2.0)
        return out.reshape(T, W), None
    g = O.log_decay(host(decay)[0], host(block.decay_bias), host(block.decay_scale_log), H).reshape(1, T, H, D)
    sb, beta = O.write_gates(gates[:, :W], gates[:, W:2 * W], bf16=True)
    k_til = O.bf16_round(sb.reshape(1, T, H, D) * O.l2norm(k, 1e-6, out_bf16=True)[0])
    read, final = O.token_memory_packed(q_hat, k_til, v, g, beta.reshape(1, T, H, D), rs, host(write_states),
                                        erase=None, lengths=lengths, scale=scale,
                                        chunk_tokens=block.chunk_tokens)
    out = O.rms_norm_gated(read.reshape(T * H, D), gate, wn, eps=1e-6, softcap=2.0)
    return out.reshape(T, W), final


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("commit", [False, True])
def test_block_packed(dev, commit, fused):
    print(f"block packed commit={commit} fused={fused}", flush=True)
    cfg = _config()
    block = _block(dev, cfg)
    block.fused_prologue = fused
    lengths = [150, 1, 300]
    T = sum(lengths)
    g = torch.Generator().manual_seed(5)
    hidden = torch.randn(T, cfg.hidden_size, generator=g).to(dev, torch.bfloat16)
    rs = (torch.randn(3, 2, 128, 128, generator=g) * 0.05).to(dev)
    ws = (torch.randn(3, 2, 128, 128, generator=g) * 0.05).to(dev)
    out, final = block.packed(hidden, rs, lengths=lengths, commit=commit, write_states=ws)
    out_ref, final_ref = _oracle_packed(block, hidden, rs, lengths, commit, ws)
    assert out.shape == (T, 256) and out.dtype == torch.bfloat16
    assert O.parity_err(host(out), out_ref, out_bf16=True) <= TOL
    if commit:
        assert O.max_rel_err(host(final), final_ref) <= TOL
    else:
        assert final is None


def test_runtime_step_on_gpu_slots(dev):
    """A step with two queries and two commits through the serving caller on
    GPU slots: residual rows and slot updates equal direct packed() calls."""
    print("runtime step on gpu slots", flush=True)
    cfg = _config(chunk_tokens=64)
    block = _block(dev, cfg, seed=3)
    g = torch.Generator().manual_seed(9)
    pool = types.SimpleNamespace(storage={0: (torch.randn(6, 1, 2, 128, 128, generator=g) * 0.05).to(dev)})
    before = pool.storage[0].clone()
    plan = plan_of([(MemoryRequest("c1", "a", "commit"), 70), (MemoryRequest("q1", "b", "query"), 1),
                    (MemoryRequest("q2", "c", "query"), 5), (MemoryRequest("c2", "d", "commit"), 20)])
    slot_of = {"c1": 4, "q1": 0, "q2": 1, "c2": 5}
    hidden = torch.randn(plan.token_count, cfg.hidden_size, generator=g).to(dev, torch.bfloat16)
    out = torch.empty_like(hidden)
    rt = MemoryRuntime(pool)
    rt.begin(plan, slot_of=slot_of, memory_read={"a": True, "b": True, "c": False, "d": True})
    rt.run_layer(0, hidden, out, block)
    rt.finish(True)
    # queries: only q1 reads (c has memory_read off)
    rq, _ = block.packed(hidden[70:71], before[0].view(1, 2, 128, 128), lengths=[1], commit=False,
                         write_states=before[0].view(1, 2, 128, 128))
    cs = torch.cat([before[4], before[5]])
    rc, fc = block.packed(torch.cat([hidden[0:70], hidden[76:96]]), cs, lengths=[70, 20], commit=True,
                          write_states=cs)
    torch.cuda.synchronize()
    assert torch.equal(out[70:71], rq)
    assert torch.equal(out[71:76], torch.zeros_like(out[71:76]))
    assert torch.equal(out[0:70], rc[:70]) and torch.equal(out[76:96], rc[70:])
    assert torch.equal(pool.storage[0][4, 0], fc[0]) and torch.equal(pool.storage[0][5, 0], fc[1])
    assert torch.equal(pool.storage[0][:4], before[:4])


@pytest.mark.parametrize("D,lengths", [(128, [150, 1, 300]), (64, [40, 700]), (256, [90, 130]), (512, [70, 1, 100])])
def test_fused_prologue_update(dev, D, lengths):
    """The update from raw projections (prologue in the WY kernel) against the
    prologue kernel followed by token_memory_packed, and against the oracle;
    the slot form on the same inputs gives the same bits."""
    print(f"fused prologue D={D} lengths={lengths}", flush=True)
    H = 2
    T = sum(lengths)
    q, k, decay, bias, rate, erase, write = _fused_rows(T, H, D, dev, seed=40 + D)
    v = (torch.randn(T, 3 * H * D, device=dev) * 1.0).to(torch.bfloat16)[:, 2 * H * D:]
    gen = torch.Generator(device=dev).manual_seed(41)
    rs = torch.randn(len(lengths), H, D, D, generator=gen, device=dev) * 0.05
    ws = torch.randn(len(lengths), H, D, D, generator=gen, device=dev) * 0.05
    read, final = memt_gdn2.token_memory_packed_fused(q, k, v, decay, bias, rate, erase, write, rs, ws,
                                                      lengths=lengths, scale=D ** -0.5, chunk_tokens=256,
                                                      num_heads=H)
    q_hat, k_til, beta, g = memt_gdn2.memory_prologue(q, k, decay, bias, rate, erase, write, H)
    read2, final2 = memt_gdn2.token_memory_packed(q_hat, k_til, v.reshape(1, T, H, D), g, beta, rs, ws, erase=None,
                                                  lengths=lengths, scale=D ** -0.5, chunk_tokens=256)
    assert O.parity_err(host(read), host(read2), out_bf16=True) <= 1e-3
    assert O.max_rel_err(host(final), host(final2)) <= 1e-3
    # the oracle from the same projections
    g_ref, sb_ref, beta_ref = _ref_gates(decay, bias, rate, erase, write, H)
    qh = O.l2norm(host(q).reshape(1, T, H, D), 1e-6, out_bf16=True)[0]
    kt = O.bf16_round(sb_ref.reshape(1, T, H, D) * O.l2norm(host(k).reshape(1, T, H, D), 1e-6, out_bf16=True)[0])
    r_ref, f_ref = O.token_memory_packed(qh, kt, host(v).reshape(1, T, H, D), g_ref.reshape(1, T, H, D),
                                         beta_ref.reshape(1, T, H, D), host(rs), host(ws), erase=None,
                                         lengths=lengths, scale=D ** -0.5, chunk_tokens=256)
    assert O.max_rel_err(host(final), f_ref) <= TOL
    assert O.parity_err(host(read), r_ref, out_bf16=True) <= TOL
    pool = torch.zeros(len(lengths) + 3, H, D, D, device=dev)
    slots_w = [len(lengths) + 2 - i for i in range(len(lengths))]
    slots_r = list(range(len(lengths)))
    pool[slots_w] = ws
    pool[slots_r] = rs
    read3 = memt_gdn2.token_memory_packed_fused_slots(q, k, v, decay, bias, rate, erase, write, pool, slots_r,
                                                      slots_w, lengths=lengths, scale=D ** -0.5, chunk_tokens=256,
                                                      num_heads=H)
    torch.cuda.synchronize()
    assert torch.equal(read3, read) and torch.equal(pool[slots_w], final)
