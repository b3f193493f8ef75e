"""Seeded random shapes through ``chunk_gdn2`` against the fp64 token
recurrence: sequence counts and lengths (ragged, some shorter than a chunk),
head counts, every head dim, output modes, write-gate dtypes, an optional
erase gate and initial state, and the write-event cuts of ``chunk_tokens``.
Each case prints its parameters first, so a failure names its case."""

import numpy as np
import pytest

from oracle import gdn2 as O
from gpu_util import bf, host, to_dev

import memt_gdn2

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _cases(n=24, seed=20261207):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([64, 128, 256, 512]))
        modes = ["snapshot", "none"] if D == 512 else ["causal", "snapshot", "none"]
        n_seq = int(rng.integers(1, 4))
        lengths = [int(x) for x in rng.integers(1, 260 if D >= 256 else 400, n_seq)]
        out.append(dict(i=i, D=D, H=int(rng.integers(1, 4)), lengths=lengths, mode=str(rng.choice(modes)),
                        beta_bf16=bool(rng.integers(0, 2)), erase=bool(rng.integers(0, 2)),
                        h0=bool(rng.integers(0, 2)), chunk_tokens=[None, 96, 128][int(rng.integers(0, 3))]))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"c{c['i']}")
def test_random_shape_vs_recurrence(dev, case):
    print(f"random case {case}", flush=True)
    D, H, lengths = case["D"], case["H"], case["lengths"]
    T = sum(lengths)
    cu = [0, *np.cumsum(lengths).tolist()]
    inp = O.synth_inputs(T, H, D, D, seed=700 + case["i"], h0_std=0.05 if case["h0"] else 0.0, n_seq=len(lengths))
    rng = np.random.default_rng(800 + case["i"])
    beta = O.bf16_round(inp["beta"]) if case["beta_bf16"] else inp["beta"]
    b = O.bf16_round(rng.uniform(0.3, 1.0, (1, T, H, D)).astype(np.float32)) if case["erase"] else None
    q, k, v, g = bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev)
    beta_d = bf(beta, dev) if case["beta_bf16"] else to_dev(beta, dev)
    h0 = to_dev(inp["h0"], dev) if case["h0"] else None
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta_d, b=bf(b, dev) if b is not None else None, initial_state=h0,
                                 cu_seqlens=cu, out_mode=case["mode"], chunk_tokens=case["chunk_tokens"])
    mode = "snapshot" if case["mode"] == "none" else case["mode"]
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], beta, b=b,
                                    h0=inp["h0"] if case["h0"] else None, cu_seqlens=cu, out_mode=mode)
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    if case["mode"] == "none":
        assert o is None
    else:
        assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL
