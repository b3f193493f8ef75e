"""GPU parity of the update at d = 256 (the wide-state Flash-like shape): the
scan then carries the state in 64-column slices, four workgroups per head.

Small cases compare with the fp64 token recurrence; long sequences with slow
decay take the two-level scan; the full wide-state workload (B=1, H=64,
T=16384, d=256) is checked on two heads against the fp64 chunked torch
oracle, and its batch-32 decode readout against the oracle readout."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, check, host, to_dev

import memt_gdn2

pytestmark = pytest.mark.gpu
TOL = 2e-3  # max|x - ref| / max|ref| (bf16 outputs: beyond one bf16 ulp of ref)
D = 256


def _dev(inp, dev):
    return (bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev),
            to_dev(inp["beta"], dev), to_dev(inp["h0"], dev))


@pytest.mark.parametrize("T", [1, 64, 200])
@pytest.mark.parametrize("mode", ["causal", "snapshot"])
def test_wide_vs_recurrent(dev, T, mode):
    print(f"wide recurrent T={T} {mode}", flush=True)
    H = 2
    inp = O.synth_inputs(T, H, D, D, seed=400 + T, h0_std=0.05)
    q, k, v, g, beta, h0 = _dev(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode=mode)
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], h0=inp["h0"],
                                    out_mode=mode)
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_wide_varlen_erase_events(dev):
    print("wide varlen erase events", flush=True)
    T, H = 300, 2
    cu = [0, 37, 167, T]
    inp = O.synth_inputs(T, H, D, D, seed=410, h0_std=0.1, n_seq=3)
    rng = np.random.default_rng(411)
    beta = O.bf16_round(inp["beta"])
    b = O.bf16_round(rng.uniform(0.3, 1.0, (1, T, H, D)).astype(np.float32))
    q, k, v, g, _, h0 = _dev(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, bf(beta, dev), b=bf(b, dev), initial_state=h0, cu_seqlens=cu,
                                 out_mode="causal", chunk_tokens=96)
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], beta, b=b, h0=inp["h0"],
                                    cu_seqlens=cu)
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_wide_token_memory_packed(dev):
    print("wide token_memory_packed", flush=True)
    T, H = 260, 2
    lengths = [130, 1, 129]
    inp = O.synth_inputs(T, H, D, D, seed=420, h0_std=0.05, n_seq=3)
    rs = (np.random.default_rng(421).standard_normal((3, H, D, D)) * 0.05).astype(np.float32)
    q, k, v, g, _, ws = _dev(inp, dev)
    beta = O.bf16_round(inp["beta"])
    read, final = memt_gdn2.token_memory_packed(q, k, v, g, bf(beta, dev), to_dev(rs, dev), ws, erase=None,
                                                lengths=lengths, scale=D ** -0.5, chunk_tokens=64)
    r_ref, f_ref = O.token_memory_packed(inp["q"], inp["k"], inp["v"], inp["g"], beta, rs, inp["h0"], erase=None,
                                         lengths=lengths, scale=D ** -0.5, chunk_tokens=64)
    assert O.max_rel_err(host(final), f_ref) <= TOL
    assert O.parity_err(host(read), r_ref, out_bf16=True) <= TOL


@pytest.mark.parametrize("mode", ["causal", "snapshot"])
def test_wide_long_memory_grouped(dev, mode):
    """One 4096-token sequence, slow decay: 64 chunks in groups of 4."""
    print(f"wide long memory {mode}", flush=True)
    T, H = 4096, 1
    inp = O.synth_inputs(T, H, D, D, seed=430, h0_std=0.05)
    inp["g"] = np.random.default_rng(431).uniform(-0.01, 0.0, inp["g"].shape).astype(np.float32)
    q, k, v, g, beta, h0 = _dev(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode=mode)
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], h0=inp["h0"],
                                    out_mode=mode)
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_wide_wy_stage_and_fwd_h(dev):
    """chunk_gdn2_fwd_intra at d = 256 against the oracle's WY quantities, and
    memt_gdn2_fwd_h of the oracle's WY tensors against the oracle scan."""
    print("wide wy stage and fwd_h", flush=True)
    T, H = 150, 2
    inp = O.synth_inputs(T, H, D, D, seed=440, h0_std=0.05)
    gk = O.chunk_local_cumsum(inp["g"], 64, scale=O.RCP_LN2).astype(np.float32)
    q, k, v, _, beta, h0 = _dev(inp, dev)
    w, u, qg, kg, Aqk, Akk = memt_gdn2.chunk_gdn2_fwd_intra(q, k, v, to_dev(gk, dev), None, beta, D ** -0.5,
                                                            disable_recompute=True)
    w, u, kg, Akk = (host(x) for x in (w, u, kg, Akk))
    wr, ur, kr = (np.zeros_like(inp[n]) for n in ("k", "v", "k"))
    for h in range(H):
        for c0 in range(0, T, 64):
            c1 = min(c0 + 64, T)
            wy = O.wy_chunk(inp["k"][0, c0:c1, h], inp["v"][0, c0:c1, h], gk[0, c0:c1, h].astype(np.float64),
                            inp["beta"][0, c0:c1, h])
            assert O.parity_err(Akk[0, c0:c1, h, :c1 - c0], wy["A"], out_bf16=True) <= TOL
            assert O.parity_err(w[0, c0:c1, h], wy["W"], out_bf16=True) <= TOL
            assert O.parity_err(u[0, c0:c1, h], wy["U"], out_bf16=True) <= TOL
            assert O.parity_err(kg[0, c0:c1, h], wy["kg"], out_bf16=True) <= TOL
            wr[0, c0:c1, h], ur[0, c0:c1, h], kr[0, c0:c1, h] = wy["W"], wy["U"], wy["kg"]
    wr, ur, kr = (O.bf16_round(x) for x in (wr, ur, kr))
    cu = [0, T]
    plan = memt_gdn2.build_chunk_plan(cu, cu, device=dev)
    snaps, final = memt_gdn2.memt_gdn2_fwd_h(bf(kr, dev), bf(wr, dev), bf(ur, dev), to_dev(gk, dev), plan,
                                             initial_state=h0)
    _, f_ref = O.state_scan(kr, wr, ur, gk, O.build_chunk_plan(cu, cu), h0=inp["h0"])
    assert O.max_rel_err(host(final), f_ref) <= TOL


def test_wide_state_full_workload(dev):
    """B=1, H=64, T=16384, d=256, chunk 64 (state 64 x 256 x 256 fp32), then a
    batch-32 decode readout over the resulting states plus 31 others."""
    from oracle.gdn2_torch import chunked_gdn2_torch, readout_torch

    T, H = 16384, 64
    print(f"wide-state workload T={T} H={H} D={D}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(20261205)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(1, T, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    k = nrm(torch.randn(1, T, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    v = torch.randn(1, T, H, D, generator=gen, device=dev).to(torch.bfloat16)
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, H, D, generator=gen, device=dev))
    beta = torch.sigmoid(torch.randn(1, T, H, D, generator=gen, device=dev))
    h0 = torch.randn(1, H, D, D, generator=gen, device=dev) * 0.02
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode="causal")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o.float()).all()) and bool(torch.isfinite(ht).all())
    hs = list(range(0, H, 9))  # 8 of the 64 heads (the fp64 oracle at d=256 costs ~1 s per head)
    sl = lambda t: t[0, :, hs].double().cpu()  # noqa: E731
    o_ref, h_ref = chunked_gdn2_torch(sl(q), sl(k), sl(v), sl(g), sl(beta), h0=h0[0, hs].double().cpu(),
                                      out_mode="causal", dtype=torch.float64)
    check(f"final state (heads {hs})", host(ht[0, hs]), h_ref.numpy(), out_bf16=False)
    check("causal output (same heads)", host(o[0, :, hs]), o_ref.numpy(), out_bf16=True)

    B = 32
    states = torch.cat([ht, torch.randn(B - 1, H, D, D, generator=gen, device=dev) * 0.02])
    qd = nrm(torch.randn(B, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    gate = torch.randn(B, H, D, generator=gen, device=dev).to(torch.bfloat16)
    wn = (1 + 0.1 * torch.randn(D, generator=gen, device=dev)).to(torch.bfloat16)
    out = memt_gdn2.readout_fused(states, qd, gate, wn, scale=D ** -0.5, eps=1e-6)
    ref = O.readout_fused(host(states), host(qd), host(gate), host(wn), scale=D ** -0.5, eps=1e-6)
    check("batch-32 readout", host(out), ref.reshape(B, H * D), out_bf16=True)
