"""GPU parity of the update on long sequences with slow decay (g in [-0.01, 0)),
where the state carries across many chunks.  These shapes take the two-level
scan (groups of chunks: per-group transitions, a serial combine over groups,
then the scan per group), so they pin the group transitions and the combine
against the fp64 token recurrence of the oracle."""

import numpy as np
import pytest

from oracle import gdn2 as O
from gpu_util import bf, host, to_dev

import memt_gdn2

pytestmark = pytest.mark.gpu
TOL = 2e-3  # max|x - ref| / max|ref| (bf16 outputs: beyond one bf16 ulp of ref)


def _slow_decay(inp, seed, lo=-0.01):
    rng = np.random.default_rng(seed)
    out = dict(inp)
    out["g"] = rng.uniform(lo, 0.0, inp["g"].shape).astype(np.float32)
    return out


def _dev(inp, dev):
    return (bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev),
            to_dev(inp["beta"], dev), to_dev(inp["h0"], dev))


@pytest.mark.parametrize("T,H,D", [(2048, 2, 128), (4096, 1, 64)])
@pytest.mark.parametrize("mode", ["causal", "snapshot"])
def test_long_memory_single_sequence(dev, T, H, D, mode):
    print(f"long memory T={T} H={H} D={D} {mode}", flush=True)
    inp = _slow_decay(O.synth_inputs(T, H, D, D, seed=300 + T + D, h0_std=0.05), seed=301)
    q, k, v, g, beta, h0 = _dev(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode=mode)
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], h0=inp["h0"],
                                    out_mode=mode)
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_long_memory_varlen_erase_events(dev):
    """Four packed sequences of uneven length (some shorter than a group),
    a channel erase gate and write events of 200 tokens."""
    T, H, D = 3000, 2, 128
    cu = [0, 700, 2300, 2400, T]
    inp = _slow_decay(O.synth_inputs(T, H, D, D, seed=310, h0_std=0.1, n_seq=4), seed=311)
    b = O.bf16_round(np.random.default_rng(312).uniform(0.3, 1.0, (1, T, H, D)).astype(np.float32))
    q, k, v, g, beta, h0 = _dev(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, b=bf(b, dev), initial_state=h0, cu_seqlens=cu,
                                 out_mode="causal", chunk_tokens=200)
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], b=b, h0=inp["h0"],
                                    cu_seqlens=cu)
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_long_memory_token_memory_packed(dev):
    """The plugin drop-in on two long requests: reads the incoming states,
    commits the update from write_states."""
    T, H, D = 2500, 2, 128
    lengths = [900, 1600]
    inp = _slow_decay(O.synth_inputs(T, H, D, D, seed=320, h0_std=0.05, n_seq=2), seed=321)
    rs = (np.random.default_rng(322).standard_normal((2, H, D, D)) * 0.05).astype(np.float32)
    q, k, v, g, _, ws = _dev(inp, dev)
    beta = O.bf16_round(inp["beta"])
    read, final = memt_gdn2.token_memory_packed(q, k, v, g, bf(beta, dev), to_dev(rs, dev), ws, erase=None,
                                                lengths=lengths, scale=D ** -0.5, chunk_tokens=256)
    r_ref, f_ref = O.token_memory_packed(inp["q"], inp["k"], inp["v"], inp["g"], beta, rs, inp["h0"], erase=None,
                                         lengths=lengths, scale=D ** -0.5, chunk_tokens=256)
    assert O.max_rel_err(host(final), f_ref) <= TOL
    assert O.parity_err(host(read), r_ref, out_bf16=True) <= TOL


def test_long_memory_fwd_h_snapshots(dev):
    """memt_gdn2_fwd_h on long reference-layout WY tensors: block snapshots in
    the middle of sequences, uncommitted events, final states."""
    T, H, D = 2000, 2, 64
    inp = _slow_decay(O.synth_inputs(T, H, D, D, seed=330, h0_std=0.05, n_seq=2), seed=331)
    samples = [0, 800, T]
    events = [0, 256, 512, 800, 1056, 1312, 1568, T]
    commit = [1, 1, 0, 1, 1, 0, 1]
    read = [0, 512, 800, 1312, T]
    gk = O.chunk_local_cumsum(inp["g"], 64, scale=O.RCP_LN2, cu_seqlens=events)
    oplan = O.build_chunk_plan(read, samples, event_slice=events, commit_mask=commit)
    w, u, kg = (np.zeros_like(inp[n]) for n in ("k", "v", "k"))
    for h in range(H):
        for c in range(oplan.num_chunk):
            c0 = int(oplan.chunk_tok0[c])
            c1 = c0 + int(oplan.chunk_len[c])
            wy = O.wy_chunk(inp["k"][0, c0:c1, h], inp["v"][0, c0:c1, h], gk[0, c0:c1, h], inp["beta"][0, c0:c1, h])
            w[0, c0:c1, h], u[0, c0:c1, h], kg[0, c0:c1, h] = wy["W"], wy["U"], wy["kg"]
    w, u, kg = (O.bf16_round(x) for x in (w, u, kg))
    gk32 = gk.astype(np.float32)
    plan = memt_gdn2.build_chunk_plan(read, samples, event_slice=events, commit_mask=commit, device=dev)
    snaps, final = memt_gdn2.memt_gdn2_fwd_h(bf(kg, dev), bf(w, dev), bf(u, dev), to_dev(gk32, dev), plan,
                                             initial_state=to_dev(inp["h0"], dev))
    s_ref, f_ref = O.state_scan(kg, w, u, gk32, oplan, h0=inp["h0"])
    assert O.max_rel_err(host(final), f_ref) <= TOL
    assert O.max_rel_err(host(snaps), s_ref) <= TOL
