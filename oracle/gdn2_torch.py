"""PyTorch-CPU port of the chunked GDN-2 update (the CPU baseline).

TEST INFRASTRUCTURE: only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` use it.  It restates the chunked WY form the reference's kernels
implement, batched over heads, in fp32 on the host cores:

* within a 64-token chunk, 16-token sub-blocks as in
  FLA/ops/gdn2/chunk_intra.py:166-417: the diagonal sub-blocks of
  ``L = (b k)(k)^T * 2^(gk_i - gk_j)`` use exact pairwise decay factors
  (FLA/ops/gdn2/chunk_intra_token_parallel.py:111-123); the off-diagonal
  sub-blocks factor the decay at the row sub-block start (chunk_intra.py:233-299);
* ``A = (I + L)^-1`` by triangular solve; ``W = A (b k 2^gk)``, ``U = A (beta v)``;
* the state scan of models/qwen/ops/_triton/state.py:76-112 and the causal
  output ``o = scale (q 2^gk) S + Aqk V_new``.

Checked against the numpy oracle (``oracle.gdn2``) in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import torch

RCP_LN2 = 1.4426950216
SUB = 16


def _scores(a, bk, gk, *, include_diag: bool):
    """``[H, C, C]`` scores ``sum_c a_ic bk_jc 2^(gk_ic - gk_jc)`` for j < i
    (j <= i with ``include_diag``), by 16-token sub-blocks."""
    H, C, K = a.shape
    out = torch.zeros(H, C, C, dtype=a.dtype)
    nsub = (C + SUB - 1) // SUB
    for I in range(nsub):
        i0, i1 = I * SUB, min(C, (I + 1) * SUB)
        gn = gk[:, i0:i0 + 1, :]  # [H,1,K] row sub-block start
        ai = a[:, i0:i1] * torch.exp2(gk[:, i0:i1] - gn)
        if I > 0:  # off-diagonal sub-blocks j < i0: both factors <= 1
            bj = bk[:, :i0] * torch.exp2(gn - gk[:, :i0])
            out[:, i0:i1, :i0] = ai @ bj.transpose(1, 2)
        # diagonal sub-block: exact pairwise factors
        d = gk[:, i0:i1, None, :] - gk[:, None, i0:i1, :]  # [H,n,n,K]
        n = i1 - i0
        mask = torch.tril(torch.ones(n, n, dtype=torch.bool), 0 if include_diag else -1)
        e = torch.where(mask[None, :, :, None], torch.exp2(torch.clamp(d, max=0.0)), torch.zeros((), dtype=a.dtype))
        out[:, i0:i1, i0:i1] = torch.einsum("hic,hjc,hijc->hij", a[:, i0:i1], bk[:, i0:i1], e)
    return out


def chunked_gdn2_torch(q, k, v, g, beta, *, b=None, h0=None, scale=None, out_mode: str = "causal",
                       chunk_size: int = 64, dtype=torch.float32):
    """One sequence: ``q,k,g [T,H,K]``, ``v,beta [T,H,V]``, ``h0 [H,K,V]`` ->
    ``(o [T,H,V], ht [H,K,V])`` in ``dtype``."""
    q, k, v, g, beta = (torch.as_tensor(x).to(dtype) for x in (q, k, v, g, beta))
    T, H, K = k.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    bk_all = k if b is None else k * torch.as_tensor(b).to(dtype)
    S = torch.zeros(H, K, V, dtype=dtype) if h0 is None else torch.as_tensor(h0).to(dtype).clone()
    S0 = S.clone()
    o = torch.zeros(T, H, V, dtype=dtype)
    for c0 in range(0, T, chunk_size):
        c1 = min(T, c0 + chunk_size)
        C = c1 - c0
        kc = k[c0:c1].transpose(0, 1)  # [H,C,K]
        bkc = bk_all[c0:c1].transpose(0, 1)
        vc = v[c0:c1].transpose(0, 1)
        bc = beta[c0:c1].transpose(0, 1)
        gk = torch.cumsum(g[c0:c1].transpose(0, 1), dim=1) * RCP_LN2  # [H,C,K]
        L = _scores(bkc, kc, gk, include_diag=False)
        eye = torch.eye(C, dtype=dtype).expand(H, C, C)
        gam = torch.exp2(gk)
        rhs = torch.cat((bkc * gam, bc * vc), dim=-1)  # [H,C,K+V]
        sol = torch.linalg.solve_triangular(eye + L, rhs, upper=False, unitriangular=True)
        W, U = sol[..., :K], sol[..., K:]
        vn = U - W @ S
        if out_mode == "causal":
            qc = q[c0:c1].transpose(0, 1)
            aqk = _scores(qc, kc, gk, include_diag=True)
            o[c0:c1] = (scale * ((qc * gam) @ S + aqk @ vn)).transpose(0, 1)
        elif out_mode == "snapshot":
            o[c0:c1] = (scale * (q[c0:c1].transpose(0, 1) @ S0)).transpose(0, 1)
        glast = gk[:, -1, :]  # [H,K]
        kg = kc * torch.exp2(glast[:, None, :] - gk)
        S = torch.exp2(glast)[:, :, None] * S + kg.transpose(1, 2) @ vn
    return o, S


def readout_torch(S, q, gate, weight, *, scale, eps, softcap=2.0, gate_kind="softcap_silu"):
    """Decode readout + MemTRMSNormGated epilogue in fp32/bf16 torch on CPU
    (models/qwen/ops/_triton/read.py:50-70, models/qwen/layer.py:22-31)."""
    r = (torch.einsum("bhk,bhkv->bhv", q.float(), S) * scale).to(torch.bfloat16).float()
    h = r * torch.rsqrt(r.pow(2).mean(-1, keepdim=True) + eps)
    h = (weight * h.to(torch.bfloat16)).float()
    gz = gate.float()
    if gate_kind == "sigmoid":
        s = torch.sigmoid(gz)
    else:
        s = softcap * torch.tanh(torch.nn.functional.silu(gz) / softcap)
    return (h * s).to(torch.bfloat16)


def recurrent_gdn2_torch(q, k, v, g, beta, *, h0=None, scale=None, dtype=torch.float32):
    """The naive token-by-token recurrence (TR Sec. 4.2, App. C eq. 22) in
    torch on the CPU, one sequence: ``q,k,g [T,H,K]``, ``v,beta [T,H,V]``,
    ``h0 [H,K,V]`` -> ``(o [T,H,V], ht [H,K,V])`` with the causal read
    ``o_t = scale q_t^T S_t``.  The reference's CPU path for the
    naive-recurrence configuration, timed as the CPU baseline."""
    q, k, v, g, beta = (x.to(dtype) for x in (q, k, v, g, beta))
    T, H, K = k.shape
    V = v.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    S = torch.zeros(H, K, V, dtype=dtype) if h0 is None else h0.to(dtype).clone()
    o = torch.empty(T, H, V, dtype=dtype)
    for t in range(T):
        S = S * torch.exp(g[t]).unsqueeze(-1)
        e = beta[t] * v[t] - torch.einsum("hk,hkv->hv", k[t], S)
        S = S + k[t].unsqueeze(-1) * e.unsqueeze(1)
        o[t] = scale * torch.einsum("hk,hkv->hv", q[t], S)
    return o, S
