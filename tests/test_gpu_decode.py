"""GPU parity of the memory blocks' decode query path (every query sample one
token long), which runs as one fused kernel: l2norm(q), the snapshot read of
each sample's state with the reference reader's bf16(S) operand, and the gated
RMSNorm.  Compared with the reference's packed() order on the oracle
(l2norm -> reader -> o_norm) from the same bf16 projection outputs, at the
decode workload's shape (64 sequences, H=16, d=128) and at the Flash head
size (d=512), on plain state batches and on pool slots."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, check, host, to_dev

import memt_gdn2
import test_gpu_block as nano
import test_gpu_flash_block as flash

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _states(n, H, D, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(n, H, D, D, generator=g, device=dev) * 0.02


def test_qwen_block_decode_batch64(dev):
    """B=64 H=16 d=128: block.packed(commit=False) with 64 one-token samples."""
    print("qwen block decode B=64 H=16 D=128", flush=True)
    cfg = nano._config(H=16, D=128, hidden=512)
    block = nano._block(dev, cfg, seed=11)
    B = 64
    g = torch.Generator(device=dev).manual_seed(12)
    hidden = torch.randn(B, cfg.hidden_size, generator=g, device=dev).to(torch.bfloat16)
    rs = _states(B, 16, 128, 13, dev)
    out, nxt = block.packed(hidden, rs, lengths=[1] * B, commit=False, write_states=rs)
    assert nxt is None and out.shape == (B, 16 * 128) and out.dtype == torch.bfloat16
    ref, _ = nano._oracle_packed(block, hidden, rs, [1] * B, False, rs)
    check("decode out (qwen, B=64)", host(out), ref, out_bf16=True)
    # the multi-token query path (l2norm -> reader -> o_norm kernels) on the same
    # inputs agrees with the fused path to the last bits but the summation order
    two = block.packed(hidden[:2], rs[:1], lengths=[2], commit=False, write_states=rs[:1])[0]
    ref2, _ = nano._oracle_packed(block, hidden[:2], rs[:1], [2], False, rs[:1])
    check("query out (qwen, one 2-token sample)", host(two), ref2, out_bf16=True)


def test_qwen_block_decode_slots(dev):
    """packed_slots(commit=False) with one-token samples reads pool[read_slot[n]]
    in place; the pool is left unchanged."""
    print("qwen block decode on slots", flush=True)
    cfg = nano._config(H=16, D=128, hidden=512)
    block = nano._block(dev, cfg, seed=21)
    B = 48
    pool = _states(80, 16, 128, 22, dev).view(80, 1, 16, 128, 128)
    before = pool.clone()
    slots = [int(x) for x in np.random.default_rng(23).permutation(80)[:B]]
    g = torch.Generator(device=dev).manual_seed(24)
    hidden = torch.randn(B, cfg.hidden_size, generator=g, device=dev).to(torch.bfloat16)
    out = block.packed_slots(hidden, pool, slots, slots, lengths=[1] * B, commit=False)
    rs = pool.view(80, 16, 128, 128)[slots]
    ref, _ = nano._oracle_packed(block, hidden, rs, [1] * B, False, rs)
    check("decode out (qwen, pool slots)", host(out), ref, out_bf16=True)
    assert torch.equal(pool, before)


def test_flash_block_decode(dev):
    """The Flash block's decode path at d=512: 64 one-token samples, H=2, on a
    state batch and on pool slots."""
    print("flash block decode B=64 H=2 D=512", flush=True)
    cfg = flash._config()
    block = flash._block(dev, cfg, seed=31)
    B = 64
    g = torch.Generator(device=dev).manual_seed(32)
    hidden = torch.randn(B, cfg.hidden_size, generator=g, device=dev).to(torch.bfloat16)
    rs = _states(B, 2, 512, 33, dev)
    out, nxt = block.packed(hidden, rs, lengths=[1] * B, commit=False, write_states=rs)
    assert nxt is None and out.shape == (B, 1024)
    ref, _ = flash._oracle_packed(block, hidden, rs, [1] * B, False, rs)
    check("decode out (flash, B=64)", host(out), ref, out_bf16=True)
    pool = _states(70, 2, 512, 34, dev)
    slots = [int(x) for x in np.random.default_rng(35).permutation(70)[:B]]
    out2 = block.packed_slots(hidden, pool, slots, slots, lengths=[1] * B, commit=False)
    ref2, _ = flash._oracle_packed(block, hidden, pool[slots], [1] * B, False, pool[slots])
    check("decode out (flash, pool slots)", host(out2), ref2, out_bf16=True)


@pytest.mark.parametrize("state_bf16", [True, False])
@pytest.mark.parametrize("D", [64, 128, 256, 512])
def test_readout_decode_op(dev, D, state_bf16):
    """The operator on raw strided q rows (a view of a fused projection) and
    strided gate rows, both gate kinds, against the oracle's l2norm, reader
    (bf16(S) or fp32 S) and gated norm."""
    print(f"readout_decode D={D} state_bf16={state_bf16}", flush=True)
    B, H = 9, 3
    rng = np.random.default_rng(40 + D)
    qkv = O.bf16_round(rng.standard_normal((B, 3 * H * D)).astype(np.float32) * 2)
    gate_rows = O.bf16_round(rng.standard_normal((B, 2 * H * D)).astype(np.float32))
    S = (rng.standard_normal((B + 4, H, D, D)) * 0.05).astype(np.float32)
    w = O.bf16_round((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    slots = rng.permutation(B + 4)[:B].astype(np.int32)
    tq, tg = bf(qkv, dev), bf(gate_rows, dev)
    q_view, g_view = tq[:, H * D:2 * H * D], tg[:, :H * D]  # strided row views, read in place
    for kind in ("softcap_silu", "sigmoid"):
        out = memt_gdn2.readout_decode(to_dev(S, dev), q_view, g_view, bf(w, dev), num_heads=H, scale=D ** -0.5,
                                       eps=1e-6, gate_kind=kind, slot_idx=torch.from_numpy(slots),
                                       state_bf16=state_bf16)
        qh = O.l2norm(qkv[:, H * D:2 * H * D].reshape(B, H, D), 1e-6, out_bf16=True)[0]
        ref = O.readout_fused(S[slots], qh, gate_rows[:, :H * D].reshape(B, H, D), w, scale=D ** -0.5, eps=1e-6,
                              gate_kind=kind, state_bf16=state_bf16).reshape(B, H * D)
        check(f"readout_decode D={D} {kind}", host(out), ref, out_bf16=True)
