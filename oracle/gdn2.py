"""CPU oracle for MemT's GDN-2 native-memory hot path (numpy).

THIS MODULE IS TEST INFRASTRUCTURE.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker (or the timed CPU baseline).  The product path (``memt_gdn2``) never
imports it and has no CPU fallback.

It restates, from the equations, what the reference computes:

* the stable gated delta rule (MemT tech report, Sec. 4.2 and App. C eq. 22;
  ``S'_t = Diag(exp g_t) S_{t-1}``, ``S_t = S'_t + k_t (beta_t*v_t - (b_t*k_t)^T S'_t)^T``)
  as a token loop (:func:`recurrent_gdn2`) and in the chunked WY form the
  reference's kernels implement (:func:`chunked_gdn2`);
* the FLA helpers on the path: ``l2norm_fwd`` and ``chunk_local_cumsum``;
* the packed chunk plan (``build_chunk_plan`` / ``packed_plan``);
* the snapshot reader and ``MemTRMSNormGated`` epilogue;
* the gate prologue of ``QwenMemoryBlock``.

All arithmetic defaults to float64.  Where the reference materialises a bf16
tensor, the optional ``rounding`` argument of :func:`chunked_gdn2` and the
``bf16`` flags of the epilogue helpers round at exactly those points, so the
oracle can also predict the reference's own rounding error.

Pinning (what checks each function beyond restating it) lives in
``tests/test_oracle.py``: recurrent == chunked (two different algorithms),
closed forms (zero keys, one-hot keys, orthonormal keys, T=1), the WY identity
``A (I + L) = I``, chunk/event-size invariance, varlen == separate runs,
torch library routines for the norms/gates, and hand-counted chunk plans.
The reference itself ships no golden vectors, known-answer tests or fixtures
for this path, so nothing reference-held pins bit-level kernel outputs.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

# FLA/ops/utils/constant.py:10 (fp32 value 0x3FB8AA3B).
RCP_LN2 = 1.4426950216
# models/common/constants.py:3
WY_TILE_TOKENS = 64

__all__ = [
    "RCP_LN2",
    "WY_TILE_TOKENS",
    "REFERENCE_ROUNDING",
    "bf16_round",
    "fp16_round",
    "l2norm",
    "chunk_local_cumsum",
    "recurrent_gdn2",
    "chunked_gdn2",
    "wy_chunk",
    "state_scan",
    "ChunkPlan",
    "build_chunk_plan",
    "packed_plan",
    "snapshot_read",
    "rms_norm_gated",
    "readout_fused",
    "log_decay",
    "write_gates",
    "token_memory_packed",
]


# ---------------------------------------------------------------------------
# bf16 emulation
# ---------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """Round to the nearest bfloat16 value (ties to even); returns float32.

    This is the conversion torch's ``.to(torch.bfloat16)`` and Triton's
    ``.to(tl.bfloat16)`` perform for finite values.
    """
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(a.shape)


def fp16_round(x) -> np.ndarray:
    """Round to the nearest IEEE binary16 value (ties to even); returns float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def _maybe_bf16(x, flag, dtype):
    """Round ``x`` when ``flag`` is set: ``True``/``"bf16"`` rounds to bfloat16,
    ``"f16"`` to binary16; a falsy flag returns ``x`` unchanged."""
    if not flag:
        return x
    if flag == "f16":
        return fp16_round(x).astype(dtype)
    return bf16_round(x).astype(dtype)


def _fmt(r, name):
    """Rounding format of quantity ``name`` under ``r`` (a set of names that
    round to bf16, or a mapping name -> "bf16" | "f16")."""
    if isinstance(r, dict):
        return r.get(name, False)
    return name in r


# ---------------------------------------------------------------------------
# FLA helpers
# ---------------------------------------------------------------------------


def l2norm(x, eps: float = 1e-6, *, out_bf16: bool = False, dtype=np.float32):
    """Row L2 normalisation over the last axis.

    FLA/modules/l2norm.py:104-106: ``rstd = 1/sqrt(sum(x*x) + eps)``;
    ``y = x * rstd`` in fp32, stored in the input dtype (bf16 on the path).
    Returns ``(y, rstd)``.
    """
    xf = np.asarray(x, dtype=dtype)
    rstd = 1.0 / np.sqrt(np.sum(xf * xf, axis=-1) + dtype(eps))
    y = xf * rstd[..., None]
    if out_bf16:
        y = bf16_round(y).astype(dtype)
    return y, rstd


def _seq_bounds(T: int, B: int, cu_seqlens):
    """(batch_row, bos, eos) triples for dense [B,T] or packed cu_seqlens input."""
    if cu_seqlens is None:
        return [(b, 0, T) for b in range(B)]
    if B != 1:
        raise ValueError("cu_seqlens requires batch size 1")
    cu = [int(c) for c in cu_seqlens]
    return [(0, cu[i], cu[i + 1]) for i in range(len(cu) - 1)]


def chunk_local_cumsum(g, chunk_size: int, *, scale=None, cu_seqlens=None, dtype=np.float64):
    """Chunk-local prefix sum along T of ``g [B,T,H,S]``, optionally scaled.

    FLA/ops/utils/cumsum.py:116-133 (vector kernel, forward, not head-first):
    every chunk of ``chunk_size`` tokens, counted from each sequence start in
    ``cu_seqlens``, restarts the sum.  The reference passes ``scale=RCP_LN2``
    so the result is in log2 units (models/qwen/ops/packed.py:50-56).
    """
    g = np.asarray(g, dtype=dtype)
    B, T = g.shape[:2]
    out = np.zeros_like(g)
    for b, bos, eos in _seq_bounds(T, B, cu_seqlens):
        for c0 in range(bos, eos, chunk_size):
            c1 = min(c0 + chunk_size, eos)
            out[b, c0:c1] = np.cumsum(g[b, c0:c1], axis=0)
    if scale is not None:
        out = out * dtype(scale)
    return out


# ---------------------------------------------------------------------------
# The recurrence (token loop)
# ---------------------------------------------------------------------------


def recurrent_gdn2(
    q,
    k,
    v,
    g,
    beta,
    *,
    b=None,
    h0=None,
    cu_seqlens=None,
    scale=None,
    out_mode: str = "causal",
    dtype=np.float64,
):
    """Naive token-by-token GDN-2 (TR Sec. 4.2; TR App. C eq. 22).

    Shapes: ``q,k,g [B,T,H,K]``, ``v,beta [B,T,H,V]``, ``b`` like ``k`` or None
    (unit erase), ``h0 [N,H,K,V]`` or None (zeros).  ``g`` is the natural-log
    decay.  Per head and token::

        S' = exp(g_t)[:,None] * S
        e  = beta_t * v_t - (b_t * k_t)^T S'
        S  = S' + k_t e^T
        o_t = scale * q_t^T S            (out_mode="causal")
        o_t = scale * q_t^T S_0          (out_mode="snapshot": MemT reads the
                                          incoming state, models/qwen/ops/packed.py:80)

    Returns ``(o [B,T,H,V], ht [N,H,K,V])``.
    """
    q, k, v, g, beta = (np.asarray(a, dtype=dtype) for a in (q, k, v, g, beta))
    bk = k if b is None else k * np.asarray(b, dtype=dtype)
    B, T, H, K = k.shape
    V = v.shape[-1]
    seqs = _seq_bounds(T, B, cu_seqlens)
    if scale is None:
        scale = K ** -0.5
    o = np.zeros((B, T, H, V), dtype=dtype)
    ht = np.zeros((len(seqs), H, K, V), dtype=dtype)
    for n, (bi, bos, eos) in enumerate(seqs):
        S = np.zeros((H, K, V), dtype=dtype) if h0 is None else np.array(h0[n], dtype=dtype)
        S0 = S.copy()
        for t in range(bos, eos):
            S = np.exp(g[bi, t])[:, :, None] * S
            e = beta[bi, t] * v[bi, t] - np.einsum("hk,hkv->hv", bk[bi, t], S)
            S = S + k[bi, t][:, :, None] * e[:, None, :]
            src = S if out_mode == "causal" else S0
            o[bi, t] = scale * np.einsum("hk,hkv->hv", q[bi, t], src)
        ht[n] = S
    return o, ht


# ---------------------------------------------------------------------------
# The chunked WY form
# ---------------------------------------------------------------------------

# Every point where the reference stores or feeds a bf16 tensor:
#   "A"     Akk inverse stored bf16 (FLA/ops/gdn2/chunk_intra.py:715-718)
#   "Aqk"   causal scores stored bf16 (chunk_intra_token_parallel.py:125-128)
#   "vb"    bf16(beta*v) operand of u (wy_fast.py:100)
#   "kb"    bf16(b*k*2^gk) operand of w (wy_fast.py:112-116,141)
#   "W","U","kg"  stored bf16 (wy_fast.py:102,139,142)
#   "S_dot" bf16(S) operand of W.S (models/qwen/ops/_triton/state.py:98)
#   "vn_dot" bf16(v_new) operand of kg^T.v_new (state.py:112)
#   "qg"    bf16 operand for the causal inter-chunk output
REFERENCE_ROUNDING = frozenset({"A", "Aqk", "vb", "kb", "W", "U", "kg", "S_dot", "vn_dot", "qg"})


def wy_chunk(k, v, gk, beta, b=None, *, rounding=frozenset(), dtype=np.float64):
    """WY quantities of ONE chunk for ONE head (FLA/ops/gdn2 intra + wy_fast).

    ``k [C,K]``, ``v,beta [C,V]``, ``gk [C,K]`` chunk-local cumulative decay in
    log2 units, ``b [C,K]`` or None.  Returns dict with

    * ``L``  strictly lower ``L[i,j] = sum_c (b k)_{i,c} k_{j,c} 2^{gk_{i,c}-gk_{j,c}}``
      (chunk_intra_token_parallel.py:111-123; chunk_intra.py:233-299),
    * ``A = (I+L)^{-1}`` (chunk_intra.py:326-395),
    * ``W = A (b*k*2^gk)``, ``U = A (beta*v)`` (wy_fast.py:92-142),
    * ``kg = k * 2^{gk_last - gk}`` (wy_fast.py:125-139),
    * ``decay = 2^{gk_last}``.
    """
    r = rounding
    k = np.asarray(k, dtype=dtype)
    bk = k if b is None else _maybe_bf16(k * np.asarray(b, dtype=dtype), _fmt(r, "kb"), dtype)
    gk = np.asarray(gk, dtype=dtype)
    C = k.shape[0]
    diff = gk[:, None, :] - gk[None, :, :]  # [i,j,c]
    tri = np.tril(np.ones((C, C), dtype=bool), -1)
    # exp2 of the masked differences only (upper entries may overflow).
    e = np.zeros_like(diff)
    e[tri] = np.exp2(diff[tri])
    L = np.einsum("ic,jc,ijc->ij", bk, k, e)
    A = np.linalg.inv(np.eye(C, dtype=dtype) + L)
    A = np.tril(A)
    A_used = _maybe_bf16(A, _fmt(r, "A"), dtype)
    gam = np.exp2(gk)
    kb = _maybe_bf16(bk * gam, _fmt(r, "kb"), dtype)
    vb = _maybe_bf16(np.asarray(beta, dtype=dtype) * np.asarray(v, dtype=dtype), _fmt(r, "vb"), dtype)
    W = _maybe_bf16(A_used @ kb, _fmt(r, "W"), dtype)
    U = _maybe_bf16(A_used @ vb, _fmt(r, "U"), dtype)
    kg = _maybe_bf16(k * np.exp2(gk[-1][None, :] - gk), _fmt(r, "kg"), dtype)
    return {"L": L, "A": A, "W": W, "U": U, "kg": kg, "decay": np.exp2(gk[-1]), "gam": gam}


def _chunks_of(bos: int, eos: int, chunk: int, chunk_tokens):
    """Token ranges of the WY chunks of one sequence: chunks of ``chunk``
    tokens inside write events of ``chunk_tokens`` tokens
    (models/qwen/ops/packed.py:16-31, layout.py:64-78)."""
    out = []
    ev = chunk_tokens if chunk_tokens else (eos - bos)
    ev = max(ev, 1)
    for e0 in range(bos, eos, ev):
        e1 = min(e0 + ev, eos)
        for c0 in range(e0, e1, chunk):
            out.append((c0, min(c0 + chunk, e1)))
    return out


def chunked_gdn2(
    q,
    k,
    v,
    g,
    beta,
    *,
    b=None,
    h0=None,
    cu_seqlens=None,
    scale=None,
    out_mode: str = "causal",
    chunk_size: int = WY_TILE_TOKENS,
    chunk_tokens=None,
    rounding=frozenset(),
    dtype=np.float64,
):
    """Chunked WY GDN-2, the form the reference's kernels implement.

    Per chunk (models/qwen/ops/_triton/state.py:76-112 for the state scan)::

        V_new = U - W . S
        o     = scale * ((q*2^gk) . S + Aqk . V_new)     (causal)
        S     = 2^{gk_last} * S + kg^T . V_new

    with ``Aqk[i,j] = sum_c q_i k_j 2^{gk_i-gk_j}`` for ``j <= i``
    (chunk_intra_token_parallel.py:120-122, diagonal included).  Chunks follow
    the reference tiling: ``chunk_size`` tokens inside write events of
    ``chunk_tokens`` tokens.  Returns ``(o, ht)`` like :func:`recurrent_gdn2`.
    """
    r = rounding
    q, k, v, g, beta = (np.asarray(a, dtype=dtype) for a in (q, k, v, g, beta))
    bb = None if b is None else np.asarray(b, dtype=dtype)
    B, T, H, K = k.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    seqs = _seq_bounds(T, B, cu_seqlens)
    o = np.zeros((B, T, H, V), dtype=dtype)
    ht = np.zeros((len(seqs), H, K, V), dtype=dtype)
    for n, (bi, bos, eos) in enumerate(seqs):
        S = np.zeros((H, K, V), dtype=dtype) if h0 is None else np.array(h0[n], dtype=dtype)
        S0 = S.copy()
        for c0, c1 in _chunks_of(bos, eos, chunk_size, chunk_tokens):
            gk = np.cumsum(g[bi, c0:c1], axis=0) * dtype(RCP_LN2)  # [C,H,K]
            for h in range(H):
                wy = wy_chunk(
                    k[bi, c0:c1, h],
                    v[bi, c0:c1, h],
                    gk[:, h],
                    beta[bi, c0:c1, h],
                    None if bb is None else bb[bi, c0:c1, h],
                    rounding=r,
                    dtype=dtype,
                )
                Sh = S[h]
                Sd = _maybe_bf16(Sh, _fmt(r, "S_dot"), dtype)
                vn = wy["U"] - wy["W"] @ Sd
                vnd = _maybe_bf16(vn, _fmt(r, "vn_dot"), dtype)
                if out_mode == "causal":
                    qh = q[bi, c0:c1, h]
                    gk_h = gk[:, h]
                    C = c1 - c0
                    diff = gk_h[:, None, :] - gk_h[None, :, :]
                    tri = np.tril(np.ones((C, C), dtype=bool))
                    e = np.zeros_like(diff)
                    e[tri] = np.exp2(diff[tri])
                    aqk = _maybe_bf16(np.einsum("ic,jc,ijc->ij", qh, k[bi, c0:c1, h], e), _fmt(r, "Aqk"), dtype)
                    qg = _maybe_bf16(qh * wy["gam"], _fmt(r, "qg"), dtype)
                    o[bi, c0:c1, h] = scale * (qg @ Sd + aqk @ vnd)
                else:
                    o[bi, c0:c1, h] = scale * (q[bi, c0:c1, h] @ S0[h])
                S[h] = wy["decay"][:, None] * Sh + wy["kg"].T @ vnd
        ht[n] = S
    return o, ht


def state_scan(kg, w, u, gk, plan, h0=None, *, dtype=np.float64):
    """Inter-chunk scan from WY tensors (models/qwen/ops/_triton/state.py:76-115).

    ``kg, w [1,T,H,K]``, ``u [1,T,H,V]``, ``gk [1,T,H,K]`` (log2 cumsum),
    ``plan`` a :class:`ChunkPlan`.  Per chunk: store the state into the
    chunk's snapshot if it starts a block; ``v_new = u - w S``; if committed,
    ``S = 2^{gk_last} S + kg^T v_new``.  Returns ``(snaps, final)``.
    """
    kg, w, u, gk = (np.asarray(a, dtype=dtype) for a in (kg, w, u, gk))
    _, T, H, K = kg.shape
    V = u.shape[-1]
    snaps = np.zeros((plan.num_block, H, K, V), dtype=dtype)
    final = np.zeros((plan.num_sample, H, K, V), dtype=dtype)
    for n in range(plan.num_sample):
        S = np.zeros((H, K, V), dtype=dtype) if h0 is None else np.array(h0[n], dtype=dtype)
        for c in range(int(plan.sample_chunk_offsets[n]), int(plan.sample_chunk_offsets[n + 1])):
            t0, ln = int(plan.chunk_tok0[c]), int(plan.chunk_len[c])
            if plan.chunk_is_block_start[c]:
                snaps[int(plan.chunk_block_ids[c])] = S
            vn = u[0, t0:t0 + ln] - np.einsum("thk,hkv->thv", w[0, t0:t0 + ln], S)
            if plan.chunk_commits[c]:
                decay = np.exp2(gk[0, t0 + ln - 1])  # [H,K]
                S = decay[:, :, None] * S + np.einsum("thk,thv->hkv", kg[0, t0:t0 + ln], vn)
        final[n] = S
    return snaps, final


# ---------------------------------------------------------------------------
# The packed chunk plan (integer work)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class ChunkPlan:
    """Restatement of models/qwen/ops/layout.py:18-44 (int64 numpy arrays)."""

    wy_tile_tokens: int
    num_event: int
    num_block: int
    num_sample: int
    num_chunk: int
    total_tokens: int
    event_slice: np.ndarray
    chunk_indices: np.ndarray
    sample_chunk_offsets: np.ndarray
    chunk_block_ids: np.ndarray
    chunk_is_block_start: np.ndarray
    chunk_tok0: np.ndarray
    chunk_len: np.ndarray
    chunk_commits: np.ndarray


def build_chunk_plan(read_slice, sample_slice, wy_tile_tokens=WY_TILE_TOKENS, *, event_slice=None, commit_mask=None):
    """Restatement of ``_build`` (models/qwen/ops/layout.py:47-108), written as
    explicit loops over events so it is independent of the reference's
    vectorised formulation."""
    read = [int(x) for x in read_slice]
    sample = [int(x) for x in sample_slice]
    event = [int(x) for x in (read_slice if event_slice is None else event_slice)]
    tok0, clen, cev, csub = [], [], [], []
    event_first_chunk = []
    for e in range(len(event) - 1):
        event_first_chunk.append(len(tok0))
        start, stop = event[e], event[e + 1]
        sub = 0
        t = start
        while t < stop:
            tok0.append(t)
            clen.append(min(wy_tile_tokens, stop - t))
            cev.append(e)
            csub.append(sub)
            sub += 1
            t += wy_tile_tokens
    num_chunk = len(tok0)
    event_first_chunk.append(num_chunk)
    # sample_chunk_offsets: first chunk of the event that starts at each sample boundary
    sample_offsets = []
    for s in sample:
        # searchsorted(event, s) (left): first event index with event[i] >= s
        i = next((j for j, ev in enumerate(event) if ev >= s), len(event))
        sample_offsets.append(event_first_chunk[i] if i < len(event_first_chunk) else num_chunk)
    block_ids, block_start = [], []
    for t in tok0:
        # searchsorted(read, t, right=True) - 1: last read boundary <= t
        blk = max(j for j, rb in enumerate(read) if rb <= t)
        block_ids.append(blk)
        block_start.append(t == read[blk])
    if commit_mask is None:
        commits = [True] * num_chunk
    else:
        cm = [bool(x) for x in commit_mask]
        commits = [cm[e] for e in cev]
    a = lambda x: np.asarray(x, dtype=np.int64)  # noqa: E731
    return ChunkPlan(
        wy_tile_tokens=wy_tile_tokens,
        num_event=len(event) - 1,
        num_block=len(read) - 1,
        num_sample=len(sample) - 1,
        num_chunk=num_chunk,
        total_tokens=event[-1],
        event_slice=a(event),
        chunk_indices=a(list(zip(cev, csub))).reshape(num_chunk, 2),
        sample_chunk_offsets=a(sample_offsets),
        chunk_block_ids=a(block_ids),
        chunk_is_block_start=a(block_start),
        chunk_tok0=a(tok0),
        chunk_len=a(clen),
        chunk_commits=a(commits),
    )


def packed_plan(lengths, *, chunk_tokens: int, wy_tile_tokens: int = WY_TILE_TOKENS):
    """Restatement of models/qwen/ops/packed.py:16-31: write events every
    ``chunk_tokens`` tokens inside each sample, every event committed."""
    samples = [0]
    for n in lengths:
        samples.append(samples[-1] + int(n))
    events = [0]
    offset = 0
    for n in lengths:
        events.extend(offset + t for t in range(chunk_tokens, int(n), chunk_tokens))
        offset += int(n)
        events.append(offset)
    return build_chunk_plan(samples, samples, wy_tile_tokens, event_slice=events, commit_mask=[True] * (len(events) - 1))


# ---------------------------------------------------------------------------
# Readout and epilogue
# ---------------------------------------------------------------------------


def snapshot_read(q, states, lengths, scale, *, state_bf16: bool = True, out_bf16: bool = True, dtype=np.float64):
    """Every token of sample n reads ``scale * q_t^T S_n``.

    models/qwen/ops/_triton/read.py:50-70: bf16(S) operand, fp32 accumulation,
    scale after the dot, bf16 output.  ``q [1,T,H,K]``, ``states [N,H,K,V]``.
    """
    q = np.asarray(q, dtype=dtype)
    S = np.asarray(states, dtype=dtype)
    if state_bf16:
        S = bf16_round(S).astype(dtype)
    out = np.zeros(q.shape[:3] + (S.shape[-1],), dtype=dtype)
    t0 = 0
    for n, ln in enumerate(lengths):
        out[0, t0 : t0 + ln] = np.einsum("thk,hkv->thv", q[0, t0 : t0 + ln], S[n]) * dtype(scale)
        t0 += ln
    if out_bf16:
        out = bf16_round(out).astype(dtype)
    return out


def _silu(x):
    return x / (1.0 + np.exp(-x))


def rms_norm_gated(x, gate, weight, *, eps: float, softcap: float = 2.0, gate_kind: str = "softcap_silu", bf16: bool = True, dtype=np.float64):
    """``MemTRMSNormGated.forward`` (models/qwen/layer.py:22-31).

    ``h = f32(x); h = h * rsqrt(mean(h^2) + eps); h = bf16(h); h = bf16(w * h);
    s = silu(f32(gate)); s = c * tanh(s / c); out = bf16(h * s)``.  With
    ``gate_kind="sigmoid"`` the gate is ``sigmoid(gate)``.  ``bf16=False``
    drops every bf16 rounding (pure float arithmetic).
    """
    h = np.asarray(x, dtype=dtype)
    var = np.mean(h * h, axis=-1, keepdims=True)
    h = h / np.sqrt(var + dtype(eps))
    h = _maybe_bf16(h, bf16, dtype)
    h = _maybe_bf16(np.asarray(weight, dtype=dtype) * h, bf16, dtype)
    gz = np.asarray(gate, dtype=dtype)
    if gate_kind == "softcap_silu":
        s = dtype(softcap) * np.tanh(_silu(gz) / dtype(softcap))
    elif gate_kind == "sigmoid":
        s = 1.0 / (1.0 + np.exp(-gz))
    else:
        raise ValueError(f"unknown gate_kind {gate_kind!r}")
    return _maybe_bf16(h * s, bf16, dtype)


def readout_fused(S, q, gate, weight, *, scale, eps, softcap=2.0, gate_kind="softcap_silu", state_bf16=False, bf16=True, dtype=np.float64):
    """Decode readout + epilogue: ``r = bf16(scale * q^T S)``, then
    :func:`rms_norm_gated`.  ``S [B,H,K,V]``, ``q,gate [B,H,K|V]``.

    The reference's reader (models/qwen/ops/_triton/read.py:64) feeds bf16(S)
    to the dot (``state_bf16=True``); the fused kernel keeps S in fp32.
    """
    Sd = np.asarray(S, dtype=dtype)
    if state_bf16:
        Sd = bf16_round(Sd).astype(dtype)
    r = np.einsum("bhk,bhkv->bhv", np.asarray(q, dtype=dtype), Sd) * dtype(scale)
    r = _maybe_bf16(r, bf16, dtype)
    return rms_norm_gated(r, gate, weight, eps=eps, softcap=softcap, gate_kind=gate_kind, bf16=bf16, dtype=dtype)


# ---------------------------------------------------------------------------
# Gate prologue
# ---------------------------------------------------------------------------


def _softplus(x):
    return np.logaddexp(0.0, x)


def log_decay(f, decay_bias, decay_scale_log, num_heads, *, dtype=np.float64):
    """``g = -exp(s_h) * softplus(f + bias)`` (models/qwen/layer.py:71-75);
    ``f [...,H*K]`` -> ``[...,H,K]``."""
    f = np.asarray(f, dtype=dtype) + np.asarray(decay_bias, dtype=dtype)
    sp = _softplus(f).reshape(*f.shape[:-1], num_heads, -1)
    return -np.exp(np.asarray(decay_scale_log, dtype=dtype))[:, None] * sp


def write_gates(erase_logits, write_logits, *, bf16: bool = True, dtype=np.float64):
    """``sqrt_erase = bf16(exp(0.5*logsigmoid(e)))``, ``write = bf16(sigmoid(w))``
    (models/qwen/layer.py:81-86)."""
    e = np.asarray(erase_logits, dtype=dtype)
    w = np.asarray(write_logits, dtype=dtype)
    logsig = -np.logaddexp(0.0, -e)
    erase = _maybe_bf16(np.exp(0.5 * logsig), bf16, dtype)
    write = _maybe_bf16(1.0 / (1.0 + np.exp(-w)), bf16, dtype)
    return erase, write


def token_memory_packed(q, k, v, log_decay_, write, read_states, write_states, *, erase, lengths, scale, chunk_tokens, rounding=frozenset(), dtype=np.float64):
    """models/qwen/ops/packed.py:34-81 end to end: every sample commits its
    tokens into ``write_states[n]`` and every token reads ``read_states[n]``.
    Returns ``(read [1,T,H,V], final [N,H,K,V])``; ``read`` follows the
    reference reader's rounding (bf16(S) operand, bf16 output)."""
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + int(n))
    _, final = chunked_gdn2(
        q, k, v, log_decay_, write, b=erase, h0=write_states, cu_seqlens=cu, scale=scale,
        out_mode="snapshot", chunk_tokens=chunk_tokens, rounding=rounding, dtype=dtype,
    )
    read = snapshot_read(q, read_states, lengths, scale, dtype=dtype)
    return read, final


def max_rel_err(x, ref) -> float:
    """``max|x - ref| / max|ref|`` (the parity metric)."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(x - ref))) / (den if den > 0 else 1.0)


def bf16_ulp(x) -> np.ndarray:
    """Spacing of bf16 values at |x| (one unit in the last place)."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(e - 7)


def parity_err(x, ref, *, out_bf16: bool) -> float:
    """The parity metric the tests assert on: ``max(|x-ref| - slack)/max|ref|``
    where ``slack`` is half a bf16 ulp of ``ref`` for bf16 outputs (the
    rounding of the output format itself: a correctly rounded bf16 result is
    that far from the exact value) and 0 for fp32 outputs."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = float(np.max(np.abs(ref))) or 1.0
    d = np.abs(x - ref)
    if out_bf16:
        d = np.maximum(d - 0.5 * bf16_ulp(ref), 0.0)
    return float(np.max(d)) / den


def parity_report(x, ref, *, out_bf16: bool) -> dict:
    """Error figures of one output tensor against its reference.

    ``max_rel``   plain ``max|x - ref| / max|ref|`` (for bf16 outputs it includes
                  the output rounding, up to 2^-9 of an element);
    ``parity``    :func:`parity_err`, the asserted metric;
    ``p99``       99th percentile over elements of ``|x - ref| / max(|ref|, f)``
                  with the floor ``f = 1e-3 max|ref|`` (elementwise relative
                  error; the floor keeps elements near zero from dividing by ~0).
    """
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if x.size == 0:
        return dict(max_rel=0.0, parity=0.0, p99=0.0)
    den = float(np.max(np.abs(ref))) or 1.0
    d = np.abs(x - ref)
    el = d / np.maximum(np.abs(ref), 1e-3 * den)
    return dict(max_rel=float(np.max(d)) / den, parity=parity_err(x, ref, out_bf16=out_bf16),
                p99=float(np.percentile(el, 99)))


def synth_inputs(T, H, K, V, *, seed, B=1, h0_std=0.0, n_seq=1, dtype=np.float32):
    """Seeded synthetic inputs with the workload's distributions:
    q,k = bf16(l2norm(N(0,1))), v = bf16(N(0,1)), g = logsigmoid(N(0,1)) fp32,
    beta = sigmoid(N(0,1)) fp32, h0 ~ N(0, h0_std^2) fp32 per sequence."""
    rng = np.random.default_rng(seed)
    q = bf16_round(l2norm(rng.standard_normal((B, T, H, K), dtype=np.float32))[0])
    k = bf16_round(l2norm(rng.standard_normal((B, T, H, K), dtype=np.float32))[0])
    v = bf16_round(rng.standard_normal((B, T, H, V), dtype=np.float32))
    g = (-np.logaddexp(0.0, -rng.standard_normal((B, T, H, K)))).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H, V))))).astype(np.float32)
    h0 = (rng.standard_normal((n_seq, H, K, V)) * h0_std).astype(np.float32)
    return dict(q=q, k=k, v=v, g=g, beta=beta, h0=h0)
