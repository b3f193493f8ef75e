"""Helpers shared by the GPU parity tests."""

import numpy as np
import torch


def to_dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(dev, dtype) if dtype is not None else t.to(dev)


def bf(a, dev):
    return to_dev(np.asarray(a, np.float32), dev, torch.bfloat16)


def host(t):
    torch.cuda.synchronize()
    return t.detach().float().cpu().numpy()


def check(name, x, ref, *, out_bf16, tol=2e-3):
    """Print the error figures of one output tensor (plain max-relative error,
    the asserted metric beyond the output's half-ulp rounding, elementwise p99)
    and assert the metric is within ``tol``."""
    from oracle import gdn2 as O

    r = O.parity_report(x, ref, out_bf16=out_bf16)
    print(f"  {name}: max_rel {r['max_rel']:.3e}  parity {r['parity']:.3e}  p99 {r['p99']:.3e}"
          f"  ({'bf16' if out_bf16 else 'fp32'}, tol {tol:g})", flush=True)
    assert r["parity"] <= tol, (name, r)
    return r


def workload_inputs(T, H, D, *, seed, h0_std=0.02):
    """Seeded CPU inputs with the workload distributions, drawn in the order
    the benchmark draws them (torch CPU generator): q, k = l2norm(N(0,1)) and
    v = N(0,1) as bf16, g = logsigmoid(N(0,1)) and beta = sigmoid(N(0,1)) fp32,
    h0 = N(0, h0_std^2) fp32 [1, H, D, D]."""
    g = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(1, T, H, D, generator=g), dim=-1).to(torch.bfloat16)
    k = nrm(torch.randn(1, T, H, D, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(1, T, H, D, generator=g).to(torch.bfloat16)
    lg = torch.nn.functional.logsigmoid(torch.randn(1, T, H, D, generator=g))
    beta = torch.sigmoid(torch.randn(1, T, H, D, generator=g))
    h0 = torch.randn(1, H, D, D, generator=g) * h0_std
    return dict(q=q, k=k, v=v, g=lg, beta=beta, h0=h0)
