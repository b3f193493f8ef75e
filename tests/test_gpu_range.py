"""GPU parity at the edges of the operand ranges.

* Large values: the update's value path (U = A beta v, the state, V_new) runs
  on f16 MFMA operands, whose range ends at 65504.  Values of |v| up to 1e5,
  heavy-tailed values and large initial states must come out right: the WY
  stage stores U in powers of two and every scan workgroup runs its columns in
  its own power-of-two scale.  Plain and two-level scans, d = 64 to 512, the
  reference-layout state scan (memt_gdn2_fwd_h) and the Flash commit path.
* Strong decay: a 16-token block whose in-block cumulative decay spans more
  than 2^96 makes the WY kernel form its diagonal tiles from exact pairwise
  factors.  g of about -8 per token on some channels reaches that branch; the
  test checks on the host that the inputs do reach it.

Every case is compared with the fp64 token recurrence (or the oracle's packed
commit) at the stated tolerance, 2e-3 of max|ref| beyond the output's
half-ulp rounding."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, check, host, to_dev

import memt_gdn2
import test_gpu_block as blk

pytestmark = pytest.mark.gpu
TOL = 2e-3
K_WIDE = 96.0  # in-block decay span (log2) beyond which the WY kernel uses exact pairwise factors


def _inputs(T, H, D, seed, *, v_scale=1.0, heavy=False, h0_std=0.05, n_seq=1, g=None):
    inp = O.synth_inputs(T, H, D, D, seed=seed, h0_std=h0_std, n_seq=n_seq)
    rng = np.random.default_rng(seed + 1)
    if heavy:
        v = rng.standard_t(1.5, size=(1, T, H, D)) * 100.0
        v = np.clip(v, -2e5, 2e5)
    else:
        v = rng.standard_normal((1, T, H, D)) * v_scale
    inp["v"] = O.bf16_round(v.astype(np.float32))
    if g is not None:
        inp["g"] = g.astype(np.float32)
    return inp


def _run_vs_recurrence(dev, inp, cu, mode, name):
    q, k, v, g, beta, h0 = (to_dev(inp[n], dev) if n in ("g", "beta", "h0") else bf(inp[n], dev)
                            for n in ("q", "k", "v", "g", "beta", "h0"))
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, cu_seqlens=cu, out_mode=mode)
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], h0=inp["h0"],
                                    cu_seqlens=cu, out_mode=mode)
    if mode == "snapshot":  # the reader's own rounding: bf16(S) operand (models/qwen/ops/_triton/read.py:64)
        bounds = cu or [0, inp["q"].shape[1]]
        o_ref = O.snapshot_read(inp["q"], inp["h0"], np.diff(bounds).tolist(), inp["q"].shape[-1] ** -0.5)
    o, ht = host(o), host(ht)
    assert np.all(np.isfinite(ht)) and np.all(np.isfinite(o)), name
    check(f"{name} final state", ht, h_ref, out_bf16=False)
    check(f"{name} output ({mode})", o, o_ref, out_bf16=True)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("case", ["v1e5", "heavy", "state1e5"])
def test_large_values(dev, D, case):
    print(f"large values D={D} case={case}", flush=True)
    T, H = 300, 2
    cu = [0, 130, T]
    kw = dict(v_scale=1e5) if case == "v1e5" else dict(heavy=True) if case == "heavy" else dict(h0_std=2e4)
    inp = _inputs(T, H, D, seed=500 + D, n_seq=2, **kw)
    assert np.max(np.abs(inp["v"])) > 6.6e4 or np.max(np.abs(inp["h0"])) > 6.6e4  # beyond the f16 range
    for mode in ("causal", "snapshot"):
        _run_vs_recurrence(dev, inp, cu, mode, f"D={D} {case}")


def test_large_values_two_level_scan(dev):
    """A long sequence takes the two-level scan: transitions, the fp32 combine
    and the per-group scan each keep their own scale."""
    print("large values, two-level scan", flush=True)
    T, H, D = 4096, 2, 64
    inp = _inputs(T, H, D, seed=600, v_scale=3e4, h0_std=1e4)
    _run_vs_recurrence(dev, inp, None, "causal", "two-level")


def test_large_values_fwd_h_import(dev):
    """memt_gdn2_fwd_h on reference-layout bf16 WY tensors whose U exceeds the f16 range."""
    print("large values, fwd_h", flush=True)
    T, H, D = 200, 2, 64
    inp = _inputs(T, H, D, seed=610, v_scale=2e5)
    gk = O.chunk_local_cumsum(inp["g"], 64, scale=O.RCP_LN2)
    w, u, kg = (np.zeros_like(inp[n]) for n in ("k", "v", "k"))
    for h in range(H):
        for c0 in range(0, T, 64):
            c1 = min(c0 + 64, T)
            wy = O.wy_chunk(inp["k"][0, c0:c1, h], inp["v"][0, c0:c1, h], gk[0, c0:c1, h], inp["beta"][0, c0:c1, h])
            w[0, c0:c1, h], u[0, c0:c1, h], kg[0, c0:c1, h] = wy["W"], wy["U"], wy["kg"]
    w, u, kg = (O.bf16_round(x) for x in (w, u, kg))
    assert np.max(np.abs(u)) > 6.6e4
    gk32 = gk.astype(np.float32)
    cu = [0, T]
    plan = memt_gdn2.build_chunk_plan(cu, cu, device=dev)
    snaps, final = memt_gdn2.memt_gdn2_fwd_h(bf(kg, dev), bf(w, dev), bf(u, dev), to_dev(gk32, dev), plan,
                                             initial_state=to_dev(inp["h0"], dev))
    _, f_ref = O.state_scan(kg, w, u, gk32, O.build_chunk_plan(cu, cu), h0=inp["h0"])
    check("fwd_h final state", host(final), f_ref, out_bf16=False)


def test_large_values_d512_commit(dev):
    """The Flash head size through token_memory_packed_flash (snapshot read,
    final states) with |v| ~ 1e5."""
    print("large values D=512", flush=True)
    T, H, D = 200, 2, 512
    lengths = [120, 80]
    inp = _inputs(T, H, D, seed=620, v_scale=1e5, n_seq=2)
    rs = (np.random.default_rng(621).standard_normal((2, H, D, D)) * 0.05).astype(np.float32)
    beta = O.bf16_round(inp["beta"])
    read, final = memt_gdn2.token_memory_packed_flash(
        bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev), bf(beta, dev),
        to_dev(rs, dev), to_dev(inp["h0"], dev), lengths=lengths, scale=D ** -0.5, chunk_tokens=64)
    r_ref, f_ref = O.token_memory_packed(inp["q"], inp["k"], inp["v"], inp["g"], beta, rs, inp["h0"], erase=None,
                                         lengths=lengths, scale=D ** -0.5, chunk_tokens=64)
    check("D=512 final state", host(final), f_ref, out_bf16=False)
    check("D=512 read", host(read), r_ref, out_bf16=True)


def _strong_decay(T, H, D, seed):
    """logsigmoid(N(0,1)) decay with a third of the channels at about -8 per token."""
    rng = np.random.default_rng(seed)
    g = -np.logaddexp(0.0, -rng.standard_normal((1, T, H, D)))
    strong = rng.random(D) < 1 / 3
    g[..., strong] = -8.0 + 0.5 * rng.standard_normal((1, T, H, int(strong.sum())))
    return np.minimum(g, 0.0)


def _max_block_span(g, cu=None, chunk=64, block=16):
    """Largest in-block cumulative decay span (log2) over the 16-token blocks
    of the 64-token chunks of each sequence in ``cu``: the WY kernel's
    condition for exact pairwise factors (each block is referenced to the
    cumulative decay at its first token)."""
    T = g.shape[1]
    cu = [0, T] if cu is None else cu
    gk = O.chunk_local_cumsum(g, chunk, scale=O.RCP_LN2, cu_seqlens=cu)
    best = 0.0
    for bos, eos in zip(cu[:-1], cu[1:]):
        for t0 in range(bos, eos, block):  # chunk starts are block starts
            t1 = min(t0 + block, eos)
            best = max(best, float(np.max(gk[0, t0] - gk[0, t0:t1])))
    return best


@pytest.mark.parametrize("D", [64, 128, 256])
def test_strong_decay_wide_blocks(dev, D):
    print(f"strong decay D={D}", flush=True)
    T, H = 200, 2
    inp = _inputs(T, H, D, seed=700 + D, g=_strong_decay(T, H, D, 701 + D))
    assert _max_block_span(inp["g"]) > K_WIDE  # the exact-factor branch runs
    for mode in ("causal", "snapshot"):
        _run_vs_recurrence(dev, inp, None, mode, f"strong decay D={D}")


def test_strong_decay_fused_d512(dev):
    """The raw-projection commit at d=512 with decay_scale_log = log(8): the
    decay g = -8 softplus(f + bias) reaches the exact-factor branch."""
    print("strong decay fused D=512", flush=True)
    H, D = 2, 512
    lengths = [90, 70]
    T = sum(lengths)
    q, k, decay, bias, rate, erase, write = blk._fused_rows(T, H, D, dev, seed=710)
    rate = torch.full_like(rate, float(np.log(8.0)))
    v = (torch.randn(T, H * D, device=dev)).to(torch.bfloat16)
    gen = torch.Generator(device=dev).manual_seed(711)
    rs = torch.randn(len(lengths), H, D, D, generator=gen, device=dev) * 0.05
    ws = torch.randn(len(lengths), H, D, D, generator=gen, device=dev) * 0.05
    read, final = memt_gdn2.token_memory_packed_fused(q, k, v, decay, bias, rate, erase, write, rs, ws,
                                                      lengths=lengths, scale=D ** -0.5, chunk_tokens=256,
                                                      num_heads=H)
    g_ref, sb_ref, beta_ref = blk._ref_gates(decay, bias, rate, erase, write, H)
    assert _max_block_span(g_ref.reshape(1, T, H, D), cu=[0, lengths[0], T]) > K_WIDE
    qh = O.l2norm(host(q).reshape(1, T, H, D), 1e-6, out_bf16=True)[0]
    kt = O.bf16_round(sb_ref.reshape(1, T, H, D) * O.l2norm(host(k).reshape(1, T, H, D), 1e-6, out_bf16=True)[0])
    r_ref, f_ref = O.token_memory_packed(qh, kt, host(v).reshape(1, T, H, D), g_ref.reshape(1, T, H, D),
                                         beta_ref.reshape(1, T, H, D), host(rs), host(ws), erase=None,
                                         lengths=lengths, scale=D ** -0.5, chunk_tokens=256)
    check("strong decay D=512 final state", host(final), f_ref, out_bf16=False)
    check("strong decay D=512 read", host(read), r_ref, out_bf16=True)
