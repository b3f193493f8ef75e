"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the oracle reproduces them on the CPU, and the HIP kernels match them on the GPU."""

from pathlib import Path

import numpy as np
import pytest

from oracle import gdn2 as O

G = Path(__file__).resolve().parent / "golden"


def _bits(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def _update():
    d = np.load(G / "gdn2_update_small.npz")
    return d, {n: _bits(d[n]) for n in ("q", "k", "v")}


def test_oracle_reproduces_update_fixture():
    d, b = _update()
    cu = d["cu_seqlens"].tolist()
    o, ht = O.recurrent_gdn2(b["q"], b["k"], b["v"], d["g"], d["beta"], h0=d["h0"], cu_seqlens=cu)
    assert np.allclose(o, d["o_causal"], rtol=1e-6, atol=1e-9) and np.allclose(ht, d["ht"], rtol=1e-6, atol=1e-9)
    o2, h2 = O.chunked_gdn2(b["q"], b["k"], b["v"], d["g"], d["beta"], h0=d["h0"], cu_seqlens=cu,
                            chunk_tokens=int(d["chunk_tokens"]))
    assert O.max_rel_err(h2, d["ht"]) < 1e-6 and O.max_rel_err(o2, d["o_causal"]) < 1e-6


def test_oracle_reproduces_readout_fixture():
    d = np.load(G / "gdn2_readout_small.npz")
    q, gate, w = (_bits(d[n]) for n in ("q", "gate", "w"))
    D = q.shape[-1]
    for kind, key in (("softcap_silu", "out_softcap"), ("sigmoid", "out_sigmoid")):
        out = O.readout_fused(d["S"], q, gate, w, scale=D ** -0.5, eps=1e-6, gate_kind=kind)
        assert np.array_equal(out.astype(np.float32), d[key])


def test_oracle_reproduces_plan_fixture():
    d = np.load(G / "plan_packed.npz")
    p = O.packed_plan(d["lengths"].tolist(), chunk_tokens=int(d["chunk_tokens"]))
    for k in d.files:
        if k not in ("lengths", "chunk_tokens"):
            assert np.array_equal(getattr(p, k), d[k]), k
    # the 3000-token sample is cut at 2048 into two write events
    assert 131 + 129 + 2048 in d["event_slice"].tolist()


@pytest.mark.gpu
def test_kernels_match_update_fixture(dev):
    import torch

    import memt_gdn2
    from gpu_util import bf, host, to_dev

    d, b = _update()
    cu = d["cu_seqlens"].tolist()
    o, ht = memt_gdn2.chunk_gdn2(bf(b["q"], dev), bf(b["k"], dev), bf(b["v"], dev), to_dev(d["g"], dev),
                                 to_dev(d["beta"], dev), initial_state=to_dev(d["h0"], dev), cu_seqlens=cu,
                                 out_mode="causal", chunk_tokens=int(d["chunk_tokens"]))
    assert O.max_rel_err(host(ht), d["ht"]) <= 2e-3
    assert O.parity_err(host(o), d["o_causal"], out_bf16=True) <= 2e-3


@pytest.mark.gpu
def test_kernels_match_readout_fixture(dev):
    import memt_gdn2
    from gpu_util import bf, host, to_dev

    d = np.load(G / "gdn2_readout_small.npz")
    q, gate, w = (_bits(d[n]) for n in ("q", "gate", "w"))
    B, H, D = q.shape
    for kind, key in (("softcap_silu", "out_softcap"), ("sigmoid", "out_sigmoid")):
        out = memt_gdn2.readout_fused(to_dev(d["S"], dev), bf(q, dev), bf(gate, dev), bf(w, dev), scale=D ** -0.5,
                                      eps=1e-6, gate_kind=kind)
        assert O.parity_err(host(out), d[key].reshape(B, H * D), out_bf16=True) <= 2e-3
