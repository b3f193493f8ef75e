"""Slot-indexed state I/O: the update and the reader working on a state pool
in place must give exactly what the gather -> compute -> write-back path of
the executor gives (runtime/executor.py:83-110), including when a commit's
final state goes to the slot it reads and starts from, on the plain scan and
on the two-level scan."""

import types

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, check, host, to_dev

import memt_gdn2
from memt_gdn2.runtime import MemoryRequest, MemoryRuntime, plan_of

pytestmark = pytest.mark.gpu


def _inputs(T, H, D, seed, dev, slow=False):
    inp = O.synth_inputs(T, H, D, D, seed=seed)
    if slow:
        inp["g"] = np.random.default_rng(seed + 1).uniform(-0.01, 0.0, inp["g"].shape).astype(np.float32)
    return (bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev),
            bf(O.bf16_round(inp["beta"]), dev))


@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("lengths,in_place", [([130, 1, 129], False), ([130, 1, 129], True),
                                              ([3000, 2900], True), ([3000, 2900], False)])
def test_packed_slots_match_gather_path(dev, D, lengths, in_place):
    print(f"packed slots D={D} lengths={lengths} in_place={in_place}", flush=True)
    H, N = 2, len(lengths)
    T = sum(lengths)
    q, k, v, g, beta = _inputs(T, H, D, seed=500 + T + D, dev=dev, slow=T > 1000)
    gen = torch.Generator(device=dev).manual_seed(7)
    pool = torch.randn(7, H, D, D, generator=gen, device=dev) * 0.05
    write_slots = [5, 0, 3][:N]
    read_slots = write_slots if in_place else [2, 6, 4][:N]
    before = pool.clone()
    read_ref, final_ref = memt_gdn2.token_memory_packed(
        q, k, v, g, beta, before[read_slots], before[write_slots], erase=None, lengths=lengths, scale=D ** -0.5,
        chunk_tokens=2048)
    read = memt_gdn2.token_memory_packed_slots(q, k, v, g, beta, pool, read_slots, write_slots, erase=None,
                                               lengths=lengths, scale=D ** -0.5, chunk_tokens=2048)
    torch.cuda.synchronize()
    assert torch.equal(read, read_ref)
    assert torch.equal(pool[write_slots], final_ref)
    untouched = [s for s in range(7) if s not in write_slots]
    assert torch.equal(pool[untouched], before[untouched])


def test_read_slots_match_gather(dev):
    H, D = 2, 128
    lengths = [40, 1, 90]
    T = sum(lengths)
    q = torch.nn.functional.normalize(torch.randn(1, T, H, D, device=dev), dim=-1).to(torch.bfloat16)
    pool = torch.randn(5, H, D, D, device=dev) * 0.1
    slots = [4, 1, 2]
    ref = memt_gdn2.snapshot_read(q, pool[slots], lengths, D ** -0.5, bf16_accumulator_output=True)
    out = memt_gdn2.read_slots(q, pool, slots, lengths, D ** -0.5)
    assert torch.equal(out, ref)
    with pytest.raises(ValueError):
        memt_gdn2.read_slots(q, pool, [4, 1, 5], lengths, D ** -0.5)  # slot out of range


def test_packed_slots_rejects_shared_final_slot(dev):
    q, k, v, g, beta = _inputs(20, 2, 64, seed=9, dev=dev)
    pool = torch.zeros(3, 2, 64, 64, device=dev)
    with pytest.raises(ValueError):
        memt_gdn2.token_memory_packed_slots(q, k, v, g, beta, pool, [0, 1], [2, 2], erase=None, lengths=[10, 10],
                                            scale=0.125, chunk_tokens=64)


def test_runtime_slot_io_matches_gather_path(dev):
    from memt_gdn2.block import QwenMemoryBlock

    cfg = types.SimpleNamespace(hidden_size=256, num_heads=2, head_dim=128, chunk_tokens=64, rms_norm_eps=1e-6,
                                output_gate_softcap=2.0)
    torch.manual_seed(11)
    block = QwenMemoryBlock(cfg, device=dev)
    with torch.no_grad():
        for name, p in block.named_parameters():
            p.copy_((torch.randn_like(p, dtype=torch.float32) * (p.shape[-1] ** -0.5 if p.ndim == 2 else 0.5))
                    + (1.0 if name == "o_norm.weight" else 0.0))
    gen = torch.Generator(device=dev).manual_seed(12)
    storage0 = torch.randn(6, 1, 2, 128, 128, generator=gen, device=dev) * 0.05
    plan = plan_of([(MemoryRequest("c1", "a", "commit"), 70), (MemoryRequest("q1", "b", "query"), 3),
                    (MemoryRequest("c2", "d", "commit"), 150)])
    slot_of = {"c1": 4, "q1": 0, "c2": 5}
    hidden = torch.randn(plan.token_count, 256, generator=gen, device=dev).to(torch.bfloat16)
    results = []
    for slot_io in (False, True):
        pool = types.SimpleNamespace(storage={0: storage0.clone()})
        rt = MemoryRuntime(pool, slot_io=slot_io)
        rt.begin(plan, slot_of=slot_of, memory_read={"a": True, "b": True, "d": True})
        out = torch.empty_like(hidden)
        rt.run_layer(0, hidden, out, block)
        rt.finish(True)
        torch.cuda.synchronize()
        results.append((out, pool.storage[0]))
    assert torch.equal(results[0][0], results[1][0])
    assert torch.equal(results[0][1], results[1][1])
    assert not torch.equal(results[1][1][4], storage0[4])  # the commit did write its slot


@pytest.mark.parametrize("lengths,in_place", [([130, 1, 129], True), ([130, 1, 129], False), ([2100, 1900], True)])
def test_slot_paths_against_the_oracle(dev, lengths, in_place):
    """The slot-indexed update and reader pinned directly against the fp64
    oracle's packed commit (models/qwen/ops/packed.py:34-81) on the same slot
    contents: reads from pool[read_slots], scans from pool[write_slots], final
    states into pool[write_slots] (in place when they are the read slots too)."""
    print(f"slot paths vs oracle lengths={lengths} in_place={in_place}", flush=True)
    H, D, N = 2, 128, len(lengths)
    T = sum(lengths)
    inp = O.synth_inputs(T, H, D, D, seed=800 + T)
    beta = O.bf16_round(inp["beta"])
    q, k, v, g = bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev)
    pool_h = (np.random.default_rng(801).standard_normal((6, H, D, D)) * 0.05).astype(np.float32)
    pool = to_dev(pool_h, dev)
    write_slots = [4, 0, 2][:N]
    read_slots = write_slots if in_place else [1, 5, 3][:N]
    read = memt_gdn2.token_memory_packed_slots(q, k, v, g, bf(beta, dev), pool, read_slots, write_slots, erase=None,
                                               lengths=lengths, scale=D ** -0.5, chunk_tokens=2048)
    r_ref, f_ref = O.token_memory_packed(inp["q"], inp["k"], inp["v"], inp["g"], beta, pool_h[read_slots],
                                         pool_h[write_slots], erase=None, lengths=lengths, scale=D ** -0.5,
                                         chunk_tokens=2048)
    check("slot commit read", host(read), r_ref, out_bf16=True)
    check("slot commit final states", host(pool)[write_slots], f_ref, out_bf16=False)
    untouched = [s for s in range(6) if s not in write_slots]
    assert np.array_equal(host(pool)[untouched], pool_h[untouched])
    # the query reader on the updated pool against the oracle's reader
    qr = memt_gdn2.read_slots(q, pool, read_slots, lengths, D ** -0.5)
    check("slot query read", host(qr), O.snapshot_read(inp["q"], host(pool)[read_slots], lengths, D ** -0.5),
          out_bf16=True)
