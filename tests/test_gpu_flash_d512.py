"""GPU parity at d = 512, the Flash model's memory head dim
(models/deepseek/ops/packed.py:70-108): unit erase gate, every sample reads
its incoming state, the commit produces the final state.

The WY kernel runs the 512 channels in two passes of the d = 256 layout, the
scan carries 32-column state slices (plain scan, no two-level groups), and the
reader holds 16 state columns per wave in registers (read_wide_kernel).  Small cases compare with the fp64 token
recurrence; the Flash-shaped workload (H=64, d=512) is checked on two heads
against the fp64 chunked torch oracle.  d = 512 has no causal output: it is
rejected with ValueError."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, host, to_dev

import memt_gdn2

pytestmark = pytest.mark.gpu
TOL = 2e-3  # max|x - ref| / max|ref| (bf16 outputs: beyond one bf16 ulp of ref)
D = 512


def _dev(inp, dev):
    return (bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev),
            to_dev(inp["beta"], dev), to_dev(inp["h0"], dev))


@pytest.mark.parametrize("T", [1, 64, 200])
@pytest.mark.parametrize("mode", ["snapshot", "none"])
def test_d512_vs_recurrent(dev, T, mode):
    print(f"d512 recurrent T={T} {mode}", flush=True)
    H = 2
    inp = O.synth_inputs(T, H, D, D, seed=600 + T, h0_std=0.05)
    q, k, v, g, beta, h0 = _dev(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode=mode)
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], h0=inp["h0"],
                                    out_mode="snapshot")
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    if mode == "snapshot":
        assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL
    else:
        assert o is None


def test_d512_varlen_erase(dev):
    """Three sequences (one shorter than a chunk), an explicit erase gate and
    bf16 write gates."""
    print("d512 varlen erase", flush=True)
    T, H = 300, 2
    cu = [0, 37, 167, T]
    inp = O.synth_inputs(T, H, D, D, seed=610, h0_std=0.1, n_seq=3)
    rng = np.random.default_rng(611)
    beta = O.bf16_round(inp["beta"])
    b = O.bf16_round(rng.uniform(0.3, 1.0, (1, T, H, D)).astype(np.float32))
    q, k, v, g, _, h0 = _dev(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, bf(beta, dev), b=bf(b, dev), initial_state=h0, cu_seqlens=cu,
                                 out_mode="snapshot")
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], beta, b=b, h0=inp["h0"], cu_seqlens=cu,
                                    out_mode="snapshot")
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_d512_token_memory_packed_flash(dev):
    print("d512 token_memory_packed_flash", flush=True)
    T, H = 260, 2
    lengths = [130, 1, 129]
    inp = O.synth_inputs(T, H, D, D, seed=620, h0_std=0.05, n_seq=3)
    rs = (np.random.default_rng(621).standard_normal((3, H, D, D)) * 0.05).astype(np.float32)
    q, k, v, g, _, ws = _dev(inp, dev)
    beta = O.bf16_round(inp["beta"])
    read, final = memt_gdn2.token_memory_packed_flash(q, k, v, g, bf(beta, dev), to_dev(rs, dev), ws,
                                                      lengths=lengths, scale=D ** -0.5, chunk_tokens=64)
    r_ref, f_ref = O.token_memory_packed(inp["q"], inp["k"], inp["v"], inp["g"], beta, rs, inp["h0"], erase=None,
                                         lengths=lengths, scale=D ** -0.5, chunk_tokens=64)
    assert O.max_rel_err(host(final), f_ref) <= TOL
    assert O.parity_err(host(read), r_ref, out_bf16=True) <= TOL
    # the Flash reader on its own: each sample reads bf16(read_states[n])
    alone = memt_gdn2.snapshot_read(q, to_dev(rs, dev), lengths, D ** -0.5, bf16_accumulator_output=True)
    assert torch.equal(alone, read)


def test_d512_long_sequence(dev):
    """One 3000-token sequence with slow decay: 47 chunks through the plain scan."""
    print("d512 long sequence", flush=True)
    T, H = 3000, 1
    inp = O.synth_inputs(T, H, D, D, seed=630, h0_std=0.05)
    inp["g"] = np.random.default_rng(631).uniform(-0.01, 0.0, inp["g"].shape).astype(np.float32)
    q, k, v, g, beta, h0 = _dev(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode="snapshot")
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], h0=inp["h0"],
                                    out_mode="snapshot")
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_d512_wy_stage_and_fwd_h(dev):
    """chunk_gdn2_fwd_intra at d = 512 (no query: the Flash write-only intra,
    models/deepseek/ops/_triton/intra.py:391-448) against the oracle's WY
    quantities, and memt_gdn2_fwd_h of the oracle's WY tensors."""
    print("d512 wy stage and fwd_h", flush=True)
    T, H = 150, 2
    inp = O.synth_inputs(T, H, D, D, seed=640, h0_std=0.05)
    gk = O.chunk_local_cumsum(inp["g"], 64, scale=O.RCP_LN2).astype(np.float32)
    _, k, v, _, beta, h0 = _dev(inp, dev)
    w, u, qg, kg, Aqk, Akk = memt_gdn2.chunk_gdn2_fwd_intra(None, k, v, to_dev(gk, dev), None, beta, D ** -0.5)
    assert qg is None and not bool(Aqk.any())
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
    s_ref, f_ref = O.state_scan(kr, wr, ur, gk, O.build_chunk_plan(cu, cu), h0=inp["h0"])
    assert O.max_rel_err(host(final), f_ref) <= TOL
    assert O.max_rel_err(host(snaps), s_ref) <= TOL


def test_d512_readout_and_norm(dev):
    print("d512 readout", flush=True)
    B, H = 5, 3
    gen = torch.Generator(device=dev).manual_seed(650)
    S = torch.randn(B, H, D, D, generator=gen, device=dev) * 0.02
    q = torch.nn.functional.normalize(torch.randn(B, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    gate = torch.randn(B, H, D, generator=gen, device=dev).to(torch.bfloat16)
    wn = (1 + 0.1 * torch.randn(D, generator=gen, device=dev)).to(torch.bfloat16)
    for kind in ("softcap_silu", "sigmoid"):
        out = memt_gdn2.readout_fused(S, q, gate, wn, scale=D ** -0.5, eps=1e-6, gate_kind=kind)
        ref = O.readout_fused(host(S), host(q), host(gate), host(wn), scale=D ** -0.5, eps=1e-6, gate_kind=kind)
        assert O.parity_err(host(out), ref.reshape(B, H * D), out_bf16=True) <= TOL
    x = torch.randn(7 * H, D, generator=gen, device=dev).to(torch.bfloat16)
    gx = torch.randn(7 * H, D, generator=gen, device=dev).to(torch.bfloat16)
    y = memt_gdn2.rms_norm_gated(x, gx, wn, eps=1e-6)
    y_ref = O.rms_norm_gated(host(x), host(gx), host(wn), eps=1e-6)
    assert O.parity_err(host(y), y_ref, out_bf16=True) <= TOL


def test_d512_causal_rejected(dev):
    inp = O.synth_inputs(64, 1, D, D, seed=660)
    q, k, v, g, beta, _ = _dev(inp, dev)
    with pytest.raises(ValueError):
        memt_gdn2.chunk_gdn2(q, k, v, g, beta, out_mode="causal")
    with pytest.raises(ValueError):
        memt_gdn2.chunk_gdn2_fwd_intra(q, k, v, g, None, beta, D ** -0.5)


def test_d512_flash_workload(dev):
    """H=64, d=512, T=4096: one commit of the whole sequence from a random
    state, its final state checked on two heads against the fp64 chunked torch
    oracle, and its snapshot read against the oracle reader, which rounds the
    state to bf16 as the reference's does (models/deepseek/ops/read.py:19)."""
    from oracle.gdn2_torch import chunked_gdn2_torch

    T, H = 4096, 64
    print(f"d512 flash workload T={T} H={H}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(20261206)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(1, T, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    k = nrm(torch.randn(1, T, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    v = torch.randn(1, T, H, D, generator=gen, device=dev).to(torch.bfloat16)
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, H, D, generator=gen, device=dev))
    beta = torch.sigmoid(torch.randn(1, T, H, D, generator=gen, device=dev)).to(torch.bfloat16)
    h0 = torch.randn(1, H, D, D, generator=gen, device=dev) * 0.02
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode="snapshot")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o.float()).all()) and bool(torch.isfinite(ht).all())
    hs = [3, 61]
    sl = lambda t: t[0, :, hs].double().cpu()  # noqa: E731
    _, h_ref = chunked_gdn2_torch(sl(q), sl(k), sl(v), sl(g), sl(beta), h0=h0[0, hs].double().cpu(),
                                  out_mode="none", dtype=torch.float64)
    assert O.max_rel_err(host(ht[0, hs]), h_ref.numpy()) <= TOL
    o_ref = O.snapshot_read(host(q[:, :, hs]), host(h0[:, hs]), [T], D ** -0.5)
    assert O.parity_err(host(o[:, :, hs]), o_ref, out_bf16=True) <= TOL
