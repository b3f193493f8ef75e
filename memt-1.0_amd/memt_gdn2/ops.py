"""GDN-2 native-memory operators on the HIP library.

Each function keeps the name, arguments, layouts and error behaviour of the
reference operator it replaces (cited per function), so the SGLang plugin can
swap imports.  Outputs are allocated with torch on the inputs' device
(caching allocator); kernels run on torch's current stream.  There is no CPU
or PyTorch fallback: a missing library or a CPU tensor raises.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .layout import WY_TILE_TOKENS, ChunkPlan, build_chunk_plan, packed_plan, plan_from_cu_seqlens

__all__ = [
    "l2norm_fwd",
    "l2norm",
    "chunk_local_cumsum",
    "chunk_gdn2_fwd_intra",
    "memt_gdn2_fwd_h",
    "memt_gdn2_read_fwd",
    "snapshot_read",
    "token_memory_packed",
    "token_memory_packed_flash",
    "chunk_gdn2",
    "rms_norm_gated",
    "readout_fused",
    "readout_decode",
    "workspace_bytes",
    "write_gates",
    "memory_prologue",
    "token_memory_packed_slots",
    "read_slots",
    "token_memory_packed_fused",
    "token_memory_packed_fused_slots",
]

_DT = {torch.bfloat16: _lib.BF16, torch.float32: _lib.F32}
_GATES = {"softcap_silu": _lib.GATE_SOFTCAP_SILU, "silu": _lib.GATE_SOFTCAP_SILU, "sigmoid": _lib.GATE_SIGMOID}
_OUT = {"none": _lib.OUT_NONE, "snapshot": _lib.OUT_SNAPSHOT, "causal": _lib.OUT_CAUSAL}


def _contig(*ts):
    return [None if t is None else t.contiguous() for t in ts]


def workspace_bytes(num_chunk: int, H: int, K: int, V: int, out_mode: str = "snapshot", num_seq: int = 1) -> int:
    """Device workspace of one chunked update (fragments of W, kg, U, ..., and the
    group states of the two-level scan when the sequences are long)."""
    return int(_lib.load().memt_gdn2_chunk_update_workspace_size(num_chunk, num_seq, H, K, V, _OUT[out_mode]))


def _workspace(device, nbytes: int) -> torch.Tensor:
    # torch's caching allocator hands out 512-byte aligned blocks.
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
    if ws.data_ptr() % 256:
        raise RuntimeError("workspace is not 256-byte aligned")
    return ws


# ---------------------------------------------------------------------------
# FLA helpers
# ---------------------------------------------------------------------------


def l2norm_fwd(x: torch.Tensor, eps: float = 1e-6, output_dtype: torch.dtype | None = None):
    """``y = x / sqrt(sum(x^2) + eps)`` per row; returns ``(y, rstd)``
    (FLA/modules/l2norm.py:147-197, D <= 512)."""
    lib = _lib.load()
    _lib.require_gpu(x)
    shape = x.shape
    x2 = x.contiguous().view(-1, shape[-1])
    out_dtype = x.dtype if output_dtype is None else output_dtype
    if x2.dtype not in _DT or out_dtype not in _DT:
        raise ValueError("l2norm_fwd supports bf16 and fp32")
    y = torch.empty(x2.shape, dtype=out_dtype, device=x.device)
    rstd = torch.empty(x2.shape[0], dtype=torch.float32, device=x.device)
    if shape[-1] > 512:
        raise RuntimeError("This layer doesn't support feature dim >= 512 on this path.")
    _lib.check(
        lib.memt_gdn2_l2norm_fwd(x2.data_ptr(), _DT[x2.dtype], y.data_ptr(), _DT[out_dtype], rstd.data_ptr(),
                                 x2.shape[0], shape[-1], float(eps), _lib.stream_of(x.device)),
        "l2norm_fwd",
    )
    return y.view(shape), rstd.view(shape[:-1])


def l2norm(inputs: torch.Tensor) -> torch.Tensor:
    """models/qwen/ops/normalization.py:6-8."""
    return l2norm_fwd(inputs)[0]


def _dense_or_varlen_plan(B: int, T: int, device, cu_seqlens, chunk_size: int) -> ChunkPlan:
    if cu_seqlens is not None:
        if B != 1:
            raise ValueError("Only batch size 1 is supported when cu_seqlens are provided")
        return plan_from_cu_seqlens(cu_seqlens, T, device, wy_tile_tokens=chunk_size)
    cu = [b * T for b in range(B + 1)]
    return build_chunk_plan(cu, cu, chunk_size, device=device)


def chunk_local_cumsum(g: torch.Tensor, chunk_size: int, reverse: bool = False, scale: float | None = None,
                       cu_seqlens=None, head_first: bool = False, output_dtype: torch.dtype | None = torch.float,
                       chunk_indices=None, **kwargs) -> torch.Tensor:
    """Chunk-local prefix sum of ``g`` [B,T,H,S] (or [B,T,H]) along T
    (FLA/ops/utils/cumsum.py:444-486).  ``chunk_indices`` is accepted for
    signature parity; chunks are derived from ``cu_seqlens`` and ``chunk_size``."""
    lib = _lib.load()
    _lib.require_gpu(g)
    if head_first:
        raise ValueError("head_first layouts are not used by the memory path")
    if output_dtype not in (None, torch.float):
        raise ValueError("chunk_local_cumsum writes fp32")
    if chunk_size != 2 ** (chunk_size.bit_length() - 1) or chunk_size > 64:
        raise ValueError("chunk_size must be a power of 2 <= 64")
    if g.ndim == 3:
        g4 = g.unsqueeze(-1)
    elif g.ndim == 4:
        g4 = g
    else:
        raise ValueError(f"Unsupported input shape {g.shape}, which should be (B, T, H, D) or (B, T, H)")
    g4 = g4.contiguous()
    if g4.dtype not in _DT:
        raise ValueError("chunk_local_cumsum supports bf16 and fp32 inputs")
    B, T, H, S = g4.shape
    plan = _dense_or_varlen_plan(B, T, g.device, cu_seqlens, chunk_size)
    out = torch.empty(g4.shape, dtype=torch.float32, device=g.device)
    p = plan.abi()
    _lib.check(
        lib.memt_gdn2_chunk_local_cumsum(g4.data_ptr(), _DT[g4.dtype], out.data_ptr(), ctypes.byref(p), H, S,
                                         1.0 if scale is None else float(scale), int(bool(reverse)),
                                         _lib.stream_of(g.device)),
        "chunk_local_cumsum",
    )
    return out.view(g.shape)


# ---------------------------------------------------------------------------
# WY stage, state scan and snapshot reader
# ---------------------------------------------------------------------------


def _check_tokens(name, t, T, H, D):
    if t.ndim != 4 or t.shape[0] != 1 or t.shape[1] != T or t.shape[2] != H or t.shape[3] != D:
        raise ValueError(f"{name} must be [1, {T}, {H}, {D}], got {tuple(t.shape)}")


def chunk_gdn2_fwd_intra(q, k, v, gk, b, w_gate, scale, cu_seqlens=None, chunk_size: int = 64, chunk_indices=None,
                         safe_gate: bool = False, disable_recompute: bool = False):
    """WY auxiliaries of every chunk (FLA/ops/gdn2/chunk_intra.py:693-787).

    Returns ``(w, u, qg, kg, Aqk, Akk)`` in the reference layouts (bf16
    [B,T,H,*]); ``qg`` is None unless ``disable_recompute``.  ``gk`` is the
    chunk-local cumulative decay in log2 units; ``b`` may be None (unit erase).
    ``q`` may be None (the Flash write-only intra,
    models/deepseek/ops/_triton/intra.py:391-448): ``Aqk`` then stays zero.
    """
    lib = _lib.load()
    _lib.require_gpu(q, k, v, gk, b, w_gate)
    if safe_gate:
        raise ValueError("safe_gate=True is not used by the memory path")
    if chunk_size != WY_TILE_TOKENS:
        raise ValueError("chunk_size must be 64")
    B, T, H, K = k.shape
    V = v.shape[-1]
    if B != 1 and cu_seqlens is not None:
        raise ValueError("Only batch size 1 is supported when cu_seqlens are provided")
    q, k, v, gk, b, w_gate = _contig(q, k, v, gk, b, w_gate)
    plan = _dense_or_varlen_plan(B, T, k.device, cu_seqlens, chunk_size)
    dev = k.device
    w = torch.empty_like(k)
    u = torch.empty_like(v)
    kg = torch.empty_like(k)
    Aqk = torch.zeros(B, T, H, chunk_size, dtype=k.dtype, device=dev)
    Akk = torch.zeros(B, T, H, chunk_size, dtype=k.dtype, device=dev)
    if q is None and disable_recompute:
        raise ValueError("disable_recompute needs q (qg = q * 2^gk)")
    qg = torch.empty_like(q) if disable_recompute else None
    ws = _workspace(dev, workspace_bytes(plan.num_chunk, H, K, V, "causal" if q is not None else "none"))
    p = plan.abi()
    _lib.check(
        lib.memt_gdn2_wy_fwd(
            _lib.ptr(q), k.data_ptr(), v.data_ptr(), gk.data_ptr(), _lib.ptr(b), w_gate.data_ptr(), _DT[w_gate.dtype],
            ctypes.byref(p), B * T, H, K, V, float(scale), w.data_ptr(), u.data_ptr(), kg.data_ptr(),
            Akk.data_ptr(), Aqk.data_ptr() if q is not None else None, _lib.ptr(qg), ws.data_ptr(), ws.numel(),
            _lib.stream_of(dev)),
        "chunk_gdn2_fwd_intra",
    )
    return w, u, qg, kg, Aqk, Akk


def memt_gdn2_fwd_h(kg, w_wy, u_wy, gk, plan: ChunkPlan, initial_state=None, output_final_state: bool = True):
    """Scan WY tiles into fp32 snapshots and final states
    (models/qwen/ops/_triton/state.py:127-174).  Returns ``(snaps, final)``."""
    lib = _lib.load()
    _lib.require_gpu(kg, w_wy, u_wy, gk, initial_state)
    _, T, H, K = kg.shape
    V = u_wy.shape[-1]
    kg, w_wy, u_wy, gk, initial_state = _contig(kg, w_wy, u_wy, gk, initial_state)
    dev = kg.device
    snaps = torch.zeros(plan.num_block, H, K, V, dtype=torch.float32, device=dev)
    final = torch.zeros(plan.num_sample, H, K, V, dtype=torch.float32, device=dev) if output_final_state else None
    ws = _workspace(dev, workspace_bytes(plan.num_chunk, H, K, V, "none", plan.num_sample))
    p = plan.abi()
    _lib.check(
        lib.memt_gdn2_fwd_h(kg.data_ptr(), w_wy.data_ptr(), u_wy.data_ptr(), gk.data_ptr(), ctypes.byref(p), T, H, K,
                            V, _lib.ptr(initial_state), snaps.data_ptr(), _lib.ptr(final), ws.data_ptr(), ws.numel(),
                            _lib.stream_of(dev)),
        "memt_gdn2_fwd_h",
    )
    return snaps, final


def memt_gdn2_read_fwd(q: torch.Tensor, snaps: torch.Tensor, plan: ChunkPlan, scale: float,
                       out_dtype: torch.dtype) -> torch.Tensor:
    """Every token reads its block's snapshot: ``bf16(scale * q . bf16(S))``
    (models/qwen/ops/read.py:10-39)."""
    lib = _lib.load()
    _lib.require_gpu(q, snaps)
    if out_dtype != torch.bfloat16:
        raise ValueError("memt_gdn2_read_fwd writes bf16")
    _, L, H, K = q.shape
    V = snaps.shape[-1]
    q, snaps = _contig(q, snaps)
    out = torch.empty(1, L, H, V, device=q.device, dtype=out_dtype)
    p = plan.abi()
    _lib.check(
        lib.memt_gdn2_read_fwd(q.data_ptr(), snaps.data_ptr(), out.data_ptr(), ctypes.byref(p), L, H, K, V,
                               float(scale), _lib.stream_of(q.device)),
        "memt_gdn2_read_fwd",
    )
    return out


def snapshot_read(query, states, lengths, scale, *, bf16_accumulator_output: bool = False):
    """Flash reader (models/deepseek/ops/read.py:6-31) with
    ``bf16_accumulator_output=True``, the mode the Flash block uses: each
    sample's tokens read ``bf16(scale * q . bf16(S_sample))`` (fp32
    accumulation, one rounding).  The reference's ``False`` mode rounds the
    dot to bf16 before scaling; that rounding is not implemented, so ``False``
    raises rather than silently returning the one-rounding result."""
    if not bf16_accumulator_output:
        raise ValueError("snapshot_read implements bf16_accumulator_output=True only "
                         "(bf16(scale * q . bf16(S)), one rounding)")
    samples = [0]
    for n in lengths:
        samples.append(samples[-1] + int(n))
    plan = build_chunk_plan(samples, samples, device=query.device)
    return memt_gdn2_read_fwd(query, states, plan, scale, out_dtype=torch.bfloat16)


# ---------------------------------------------------------------------------
# The packed commit (plugin drop-in) and the generic chunked update
# ---------------------------------------------------------------------------


def _chunk_update(q, k, v, g, beta, b, h0, read_states, plan: ChunkPlan, scale: float, out_mode: str,
                  want_final: bool = True, snaps=None):
    lib = _lib.load()
    _lib.require_gpu(q, k, v, g, beta, b, h0, read_states)
    _, T, H, K = k.shape
    V = v.shape[-1]
    if plan.total_tokens != T:
        raise ValueError("plan does not cover the token axis")
    for name, t, D in (("k", k, K), ("v", v, V), ("log_decay", g, K), ("write", beta, V)):
        _check_tokens(name, t, T, H, D)
    if q is not None:
        _check_tokens("q", q, T, H, K)
    if b is not None:
        _check_tokens("erase", b, T, H, K)
    for name, t, dt in (("q", q, torch.bfloat16), ("k", k, torch.bfloat16), ("v", v, torch.bfloat16),
                        ("log_decay", g, torch.float32), ("erase", b, torch.bfloat16)):
        if t is not None and t.dtype != dt:
            raise ValueError(f"{name} must be {dt}, got {t.dtype}")
    if beta.dtype not in _DT:
        raise ValueError("write gate must be bf16 or fp32")
    # write states per sample, read states per read block (one per sample in
    # the packed commit, whose samples are its read blocks)
    for name, t, rows in (("write_states", h0, plan.num_sample), ("read_states", read_states, plan.num_block)):
        expected = (rows, H, K, V)
        if t is not None and (tuple(t.shape) != expected or t.dtype != torch.float32):
            raise ValueError(f"{name} must be fp32 {expected}")
    q, k, v, g, beta, b, h0, read_states = _contig(q, k, v, g, beta, b, h0, read_states)
    dev = k.device
    final = torch.empty(plan.num_sample, H, K, V, dtype=torch.float32, device=dev) if want_final else None
    o = torch.empty(1, T, H, V, dtype=torch.bfloat16, device=dev) if out_mode != "none" else None
    ws = _workspace(dev, workspace_bytes(plan.num_chunk, H, K, V, out_mode, plan.num_sample))
    p = plan.abi()
    _lib.check(
        lib.memt_gdn2_chunk_update(
            _lib.ptr(q), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), _DT[beta.dtype], _lib.ptr(b),
            _lib.ptr(h0), _lib.ptr(final), _lib.ptr(read_states), _lib.ptr(snaps), _lib.ptr(o), ctypes.byref(p), T,
            H, K, V, float(scale), _OUT[out_mode], ws.data_ptr(), ws.numel(), _lib.stream_of(dev)),
        "chunk_update",
    )
    return o, final


def token_memory_packed(q, k, v, log_decay, write, read_states, write_states, *, erase, lengths, scale,
                        chunk_tokens):
    """Commit packed samples and read each sample's incoming snapshot
    (models/qwen/ops/packed.py:34-81).

    Every sample ``n`` scans its tokens from ``write_states[n]`` (result:
    ``final[n]``) while all its tokens read ``read_states[n]``.  ``erase`` is
    the channel erase gate [1,T,H,K] bf16, or None for the unit gate the
    stable variant passes (models/qwen/layer.py:97).  Returns
    ``(read [1,T,H,V] bf16, final [N,H,K,V] fp32)``.
    """
    if not lengths or any(int(n) <= 0 for n in lengths):
        raise ValueError("Packed sample lengths must be positive")
    plan = packed_plan(lengths, k.device, chunk_tokens=chunk_tokens)
    return _chunk_update(q, k, v, log_decay, write, erase, write_states, read_states, plan, scale, "snapshot")


def token_memory_packed_flash(q, k, v, log_decay, write, read_states, write_states, *, lengths, scale,
                              chunk_tokens):
    """Flash variant (models/deepseek/ops/packed.py:70-108): unit erase gate,
    every sample reads its incoming state."""
    return token_memory_packed(q, k, v, log_decay, write, read_states, write_states, erase=None, lengths=lengths,
                               scale=scale, chunk_tokens=chunk_tokens)


def chunk_gdn2(q, k, v, g, beta, *, b=None, initial_state=None, output_final_state: bool = True, cu_seqlens=None,
               scale: float | None = None, out_mode: str = "causal", chunk_tokens=None):
    """Chunked GDN-2 over independent sequences (packed by ``cu_seqlens``).

    ``out_mode="causal"``: ``o_t = scale * q_t^T S_t``; ``"snapshot"``: every
    token reads its sequence's initial state (MemT's commit read);
    ``"none"``: state only.  Returns ``(o, ht)``.
    """
    if out_mode not in _OUT:
        raise ValueError(f"out_mode must be one of {sorted(_OUT)}")
    B, T, H, K = k.shape
    if B != 1:
        if cu_seqlens is not None:
            raise ValueError("Only batch size 1 is supported when cu_seqlens are provided")
        cu = [i * T for i in range(B + 1)]
        flat = lambda t: None if t is None else t.reshape(1, B * T, *t.shape[2:])  # noqa: E731
        o, ht = chunk_gdn2(flat(q), flat(k), flat(v), flat(g), flat(beta), b=flat(b), initial_state=initial_state,
                           output_final_state=output_final_state, cu_seqlens=cu, scale=scale, out_mode=out_mode,
                           chunk_tokens=chunk_tokens)
        return (None if o is None else o.view(B, T, H, -1)), ht
    plan = plan_from_cu_seqlens(cu_seqlens, T, k.device, chunk_tokens=chunk_tokens)
    if scale is None:
        scale = K ** -0.5
    read_states = initial_state
    if out_mode == "snapshot" and initial_state is None:
        read_states = torch.zeros(plan.num_sample, H, K, v.shape[-1], dtype=torch.float32, device=k.device)
    return _chunk_update(q if out_mode != "none" else None, k, v, g, beta, b, initial_state,
                         read_states if out_mode == "snapshot" else None, plan, scale, out_mode,
                         want_final=output_final_state)


# ---------------------------------------------------------------------------
# Readout epilogue
# ---------------------------------------------------------------------------


def rms_norm_gated(x, gate, weight, *, eps: float, softcap: float = 2.0, gate_kind: str = "softcap_silu"):
    """``MemTRMSNormGated.forward`` (models/qwen/layer.py:22-31) over the last axis."""
    lib = _lib.load()
    _lib.require_gpu(x, gate, weight)
    if gate_kind not in _GATES:
        raise ValueError(f"gate_kind must be one of {sorted(_GATES)}")
    if x.shape != gate.shape or weight.shape != (x.shape[-1],):
        raise ValueError("x/gate must match and weight must be [dim]")
    if x.dtype != torch.bfloat16 or gate.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("rms_norm_gated expects bf16 x, gate and weight")
    x2, g2, w2 = _contig(x, gate, weight)
    out = torch.empty_like(x2)
    dim = x.shape[-1]
    _lib.check(
        lib.memt_gdn2_rms_norm_gated(x2.data_ptr(), g2.data_ptr(), w2.data_ptr(), out.data_ptr(), x2.numel() // dim,
                                     dim, float(eps), float(softcap), _GATES[gate_kind], _lib.stream_of(x.device)),
        "rms_norm_gated",
    )
    return out


def readout_fused(states, q, gate, weight, *, scale: float, eps: float, softcap: float = 2.0,
                  gate_kind: str = "softcap_silu", slot_idx=None):
    """Decode readout of one query token per sequence fused with the
    epilogue: ``r = bf16(scale * q . S)`` then ``MemTRMSNormGated(r, gate)``.

    ``states`` [slots,H,K,V] fp32 (``slot_idx`` [B] int32 picks each
    sequence's slot, default ``b``), ``q`` [B,H,K] bf16 (l2-normalised by the
    caller), ``gate`` [B,H,V] bf16, ``weight`` [V] bf16.  Returns [B, H*V] bf16.
    """
    lib = _lib.load()
    _lib.require_gpu(states, q, gate, weight)
    if gate_kind not in _GATES:
        raise ValueError(f"gate_kind must be one of {sorted(_GATES)}")
    B, H, K = q.shape
    V = states.shape[-1]
    if states.ndim != 4 or states.shape[1] != H or states.shape[2] != K or states.dtype != torch.float32:
        raise ValueError("states must be fp32 [slots, H, K, V]")
    if gate.shape != (B, H, V) or weight.shape != (V,):
        raise ValueError("gate must be [B, H, V] and weight [V]")
    if slot_idx is None and states.shape[0] < B:
        raise ValueError("fewer state slots than sequences")
    if slot_idx is not None:
        if not isinstance(slot_idx, torch.Tensor) or not slot_idx.is_cuda:
            # host indices are range-checked before they reach the kernel
            host = torch.as_tensor(slot_idx, dtype=torch.int64).reshape(-1)
            if host.numel() != B or (B and (int(host.min()) < 0 or int(host.max()) >= states.shape[0])):
                raise ValueError("slot_idx must hold B indices into the state slots")
            slot_idx = host.to(device=q.device, dtype=torch.int32)
        if slot_idx.dtype != torch.int32 or slot_idx.shape != (B,):
            raise ValueError("slot_idx must be int32 [B]")
    states, q, gate, weight, slot_idx = _contig(states, q, gate, weight, slot_idx)
    out = torch.empty(B, H * V, dtype=torch.bfloat16, device=q.device)
    _lib.check(
        lib.memt_gdn2_readout_fused(states.data_ptr(), _lib.ptr(slot_idx), q.data_ptr(), gate.data_ptr(),
                                    weight.data_ptr(), out.data_ptr(), B, H, K, V, float(scale), float(eps),
                                    float(softcap), _GATES[gate_kind], _lib.stream_of(q.device)),
        "readout_fused",
    )
    return out


def readout_decode(states, q, gate, weight, *, num_heads: int, scale: float, eps: float, softcap: float = 2.0,
                   gate_kind: str = "softcap_silu", q_eps: float = 1e-6, slot_idx=None, normalize_q: bool = True,
                   state_bf16: bool = True):
    """The memory block's decode query path in one kernel: one query token per
    sample, ``q_hat = l2norm(q)``, ``r = bf16(scale * q_hat . S)`` and
    ``MemTRMSNormGated(r, gate)`` (models/qwen/layer.py:112-131 for
    length-1 samples; Flash: models/deepseek/layer.py:174-183).

    ``q`` [..., B, H*K] raw bf16 projection rows (row views of the fused QKV
    projection are read in place), ``gate`` [..., B, H*V] bf16 rows,
    ``states`` [slots, H, K, V] fp32 read at ``slot_idx[b]`` (default ``b``).
    ``state_bf16`` rounds S to bf16 inside the dot, as the reference reader
    does.  Returns [B, H*V] bf16."""
    lib = _lib.load()
    _lib.require_gpu(states, q, gate, weight)
    if gate_kind not in _GATES:
        raise ValueError(f"gate_kind must be one of {sorted(_GATES)}")
    H = num_heads
    if states.ndim != 4 or states.shape[1] != H or states.dtype != torch.float32 or not states.is_contiguous():
        raise ValueError(f"states must be contiguous fp32 [slots, {H}, K, V]")
    K, V = states.shape[2], states.shape[3]
    q2, qs = _rows(q, H * K, "q")
    g2, gs = _rows(gate, H * V, "gate")
    B = q2.shape[0]
    if g2.shape[0] != B:
        raise ValueError("q and gate must hold the same number of query rows")
    if weight.shape != (V,) or weight.dtype != torch.bfloat16:
        raise ValueError("weight must be bf16 [V]")
    if slot_idx is None:
        if states.shape[0] < B:
            raise ValueError("fewer state slots than query rows")
    else:
        slot_idx = _slot_index(slot_idx, B, states.shape[0], q.device, "slot_idx")
    flags = (_lib.READOUT_L2NORM_Q if normalize_q else 0) | (_lib.READOUT_STATE_BF16 if state_bf16 else 0)
    (weight,) = _contig(weight)
    out = torch.empty(B, H * V, dtype=torch.bfloat16, device=q.device)
    _lib.check(
        lib.memt_gdn2_readout_decode(states.data_ptr(), _lib.ptr(slot_idx), q2.data_ptr(), qs, g2.data_ptr(), gs,
                                     weight.data_ptr(), out.data_ptr(), B, H, K, V, float(scale), float(q_eps),
                                     float(eps), float(softcap), _GATES[gate_kind], flags,
                                     _lib.stream_of(q.device)),
        "readout_decode",
    )
    return out


# ---------------------------------------------------------------------------
# Gate and q/k prologue
# ---------------------------------------------------------------------------


def _rows(x: torch.Tensor, width: int, name: str):
    """``x`` as ``[T, width]`` bf16 rows with the stride the kernel reads
    (views of a fused projection keep their row stride; anything else is
    made contiguous first)."""
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bf16")
    if x.shape[-1] != width:
        raise ValueError(f"{name} must have {width} channels per token, got {tuple(x.shape)}")
    try:
        x2 = x.view(-1, width)
    except RuntimeError:
        x2 = x.reshape(-1, width).contiguous()
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16 or (x2.shape[0] > 1 and x2.stride(0) < width):
        x2 = x2.contiguous()
    return x2, (x2.stride(0) if x2.shape[0] > 1 else width)


def _gate_params(decay_bias, decay_scale_log, H: int, D: int, device):
    bias = decay_bias.reshape(-1)
    rate = decay_scale_log.reshape(-1)
    if bias.numel() != H * D or rate.numel() != H:
        raise ValueError(f"decay_bias must hold {H * D} values and decay_scale_log {H}")
    bias, rate = (t.to(device=device, dtype=torch.bfloat16).contiguous() for t in (bias, rate))
    return bias, rate


def write_gates(decay, decay_bias, decay_scale_log, erase, write, num_heads: int):
    """``QwenMemoryBlock._log_decay`` + ``_write_gates`` (models/qwen/layer.py:71-88)
    from the projection outputs: ``decay`` = f_down(decay latent) [..., T, H*D],
    ``erase`` and ``write`` logits [..., T, H*D] (bf16 views are read in place).
    Returns ``(sqrt_b [1,T,H,D] bf16, beta [1,T,H,D] bf16, g [1,T,H,D] fp32)``
    in the reference's return order (erase, write, log_decay)."""
    lib = _lib.load()
    _lib.require_gpu(decay, erase, write)
    width = decay.shape[-1]
    if width % num_heads:
        raise ValueError("decay width must be a multiple of num_heads")
    D = width // num_heads
    f2, fs = _rows(decay, width, "decay")
    e2, es = _rows(erase, width, "erase")
    w2, ws = _rows(write, width, "write")
    T = f2.shape[0]
    if e2.shape[0] != T or w2.shape[0] != T:
        raise ValueError("decay, erase and write must cover the same tokens")
    bias, rate = _gate_params(decay_bias, decay_scale_log, num_heads, D, decay.device)
    g = torch.empty(1, T, num_heads, D, dtype=torch.float32, device=decay.device)
    sqrt_b = torch.empty(1, T, num_heads, D, dtype=torch.bfloat16, device=decay.device)
    beta = torch.empty_like(sqrt_b)
    _lib.check(
        lib.memt_gdn2_write_gates(f2.data_ptr(), fs, bias.data_ptr(), rate.data_ptr(), e2.data_ptr(), es,
                                  w2.data_ptr(), ws, g.data_ptr(), sqrt_b.data_ptr(), beta.data_ptr(), T, num_heads,
                                  D, _lib.stream_of(decay.device)),
        "write_gates",
    )
    return sqrt_b, beta, g


def memory_prologue(q, k, decay, decay_bias, decay_scale_log, erase, write, num_heads: int, eps: float = 1e-6):
    """Commit-path inputs of ``QwenMemoryBlock.packed`` in one kernel
    (models/qwen/layer.py:71-97): ``q_hat = l2norm(q)``,
    ``k_til = bf16(sqrt_b * l2norm(k))``, the decay ``g`` and write gate
    ``beta``.  Raw ``q``/``k`` are [..., T, H*D] bf16 (views of the fused QKV
    projection are read in place).  Returns ``(q_hat, k_til, beta, g)`` as
    [1,T,H,D]; the update then runs with the unit erase gate (``erase=None``)."""
    lib = _lib.load()
    _lib.require_gpu(q, k, decay, erase, write)
    width = decay.shape[-1]
    if width % num_heads:
        raise ValueError("decay width must be a multiple of num_heads")
    D = width // num_heads
    q2, qs = _rows(q, width, "q")
    k2, ks = _rows(k, width, "k")
    f2, fs = _rows(decay, width, "decay")
    e2, es = _rows(erase, width, "erase")
    w2, ws = _rows(write, width, "write")
    T = f2.shape[0]
    if any(x.shape[0] != T for x in (q2, k2, e2, w2)):
        raise ValueError("q, k, decay, erase and write must cover the same tokens")
    bias, rate = _gate_params(decay_bias, decay_scale_log, num_heads, D, decay.device)
    dev = decay.device
    q_hat = torch.empty(1, T, num_heads, D, dtype=torch.bfloat16, device=dev)
    k_til = torch.empty_like(q_hat)
    beta = torch.empty_like(q_hat)
    g = torch.empty(1, T, num_heads, D, dtype=torch.float32, device=dev)
    _lib.check(
        lib.memt_gdn2_memory_prologue(q2.data_ptr(), qs, k2.data_ptr(), ks, f2.data_ptr(), fs, bias.data_ptr(),
                                      rate.data_ptr(), e2.data_ptr(), es, w2.data_ptr(), ws, q_hat.data_ptr(),
                                      k_til.data_ptr(), g.data_ptr(), beta.data_ptr(), T, num_heads, D, float(eps),
                                      _lib.stream_of(dev)),
        "memory_prologue",
    )
    return q_hat, k_til, beta, g


# ---------------------------------------------------------------------------
# Slot-indexed state I/O (the executor's gather and write-back folded in)
# ---------------------------------------------------------------------------


def _pool_view(pool: torch.Tensor, H: int, K: int, V: int) -> torch.Tensor:
    """A state pool ``[slots, H, K, V]`` (or the runtime's ``[slots, 1, H, K, V]``)
    as the contiguous fp32 ``[slots, H, K, V]`` the kernels index in place."""
    if pool.dtype != torch.float32 or not pool.is_contiguous() or pool.shape[-3:] != (H, K, V):
        raise ValueError(f"state pool must be contiguous fp32 [slots, ..., {H}, {K}, {V}]")
    return pool.view(-1, H, K, V)


def _slot_index(slots, n: int, n_slots: int, device, name: str, distinct: bool = False) -> torch.Tensor:
    """Slot indices as device int32.  Host indices are range-checked here;
    device tensors are trusted (checking them would copy them back)."""
    if isinstance(slots, torch.Tensor) and slots.is_cuda:
        if slots.dtype != torch.int32 or slots.shape != (n,):
            raise ValueError(f"{name} must be int32 [{n}]")
        return slots.contiguous()
    host = torch.as_tensor(slots, dtype=torch.int64).reshape(-1)
    if host.numel() != n or (n and (int(host.min()) < 0 or int(host.max()) >= n_slots)):
        raise ValueError(f"{name} must hold {n} indices into the {n_slots} state slots")
    if distinct and len(set(host.tolist())) != n:
        raise ValueError(f"{name} must not repeat a slot")
    return host.to(device=device, dtype=torch.int32)


def token_memory_packed_slots(q, k, v, log_decay, write, pool, read_slots, write_slots, *, erase, lengths, scale,
                              chunk_tokens):
    """``token_memory_packed`` on a state pool, in place: sample ``n`` scans
    from ``pool[write_slots[n]]``, its final state replaces that slot, and its
    tokens read ``pool[read_slots[n]]`` as it was before the call.  This is the
    executor's commit pass (runtime/executor.py:83-110) without the
    ``torch.cat`` gather and the ``index_copy_`` write-back.  Returns ``read``."""
    if not lengths or any(int(n) <= 0 for n in lengths):
        raise ValueError("Packed sample lengths must be positive")
    lib = _lib.load()
    _, T, H, K = k.shape
    V = v.shape[-1]
    _lib.require_gpu(q, k, v, log_decay, write, erase, pool)
    pv = _pool_view(pool, H, K, V)
    plan = packed_plan(lengths, k.device, chunk_tokens=chunk_tokens)
    N = plan.num_sample
    rs = _slot_index(read_slots, N, pv.shape[0], k.device, "read_slots")
    ws_ = _slot_index(write_slots, N, pv.shape[0], k.device, "write_slots", distinct=True)
    for name, t, D in (("q", q, K), ("k", k, K), ("v", v, V), ("log_decay", log_decay, K), ("write", write, V)):
        _check_tokens(name, t, T, H, D)
    if erase is not None:
        _check_tokens("erase", erase, T, H, K)
    for name, t, dt in (("q", q, torch.bfloat16), ("k", k, torch.bfloat16), ("v", v, torch.bfloat16),
                        ("log_decay", log_decay, torch.float32), ("erase", erase, torch.bfloat16)):
        if t is not None and t.dtype != dt:
            raise ValueError(f"{name} must be {dt}, got {t.dtype}")
    if write.dtype not in _DT:
        raise ValueError("write gate must be bf16 or fp32")
    q, k, v, log_decay, write, erase = _contig(q, k, v, log_decay, write, erase)
    o = torch.empty(1, T, H, V, dtype=torch.bfloat16, device=k.device)
    ws = _workspace(k.device, workspace_bytes(plan.num_chunk, H, K, V, "snapshot", N))
    p = plan.abi()
    _lib.check(
        lib.memt_gdn2_chunk_update_slots(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), log_decay.data_ptr(), write.data_ptr(), _DT[write.dtype],
            _lib.ptr(erase), pv.data_ptr(), pv.shape[0], rs.data_ptr(), ws_.data_ptr(), ws_.data_ptr(), o.data_ptr(),
            ctypes.byref(p), T, H, K, V, float(scale), _OUT["snapshot"], ws.data_ptr(), ws.numel(),
            _lib.stream_of(k.device)),
        "chunk_update_slots",
    )
    return o


def read_slots(q, pool, read_slots_, lengths, scale):
    """Every token of sample ``n`` reads ``bf16(scale * q . bf16(pool[read_slots[n]]))``
    (models/qwen/ops/read.py:10-39 on the pool in place)."""
    lib = _lib.load()
    _lib.require_gpu(q, pool)
    _, T, H, K = q.shape
    pv = _pool_view(pool, H, K, pool.shape[-1])
    V = pv.shape[-1]
    samples = [0]
    for n in lengths:
        samples.append(samples[-1] + int(n))
    if samples[-1] != T:
        raise ValueError("lengths must cover the query tokens")
    plan = build_chunk_plan(samples, samples, device=q.device)
    rs = _slot_index(read_slots_, plan.num_block, pv.shape[0], q.device, "read_slots")
    (q,) = _contig(q)
    out = torch.empty(1, T, H, V, device=q.device, dtype=torch.bfloat16)
    p = plan.abi()
    _lib.check(
        lib.memt_gdn2_read_fwd_slots(q.data_ptr(), pv.data_ptr(), pv.shape[0], rs.data_ptr(), out.data_ptr(),
                                     ctypes.byref(p), T, H, K, V, float(scale), _lib.stream_of(q.device)),
        "read_fwd_slots",
    )
    return out


# ---------------------------------------------------------------------------
# The commit path from raw projections (prologue inside the WY kernel)
# ---------------------------------------------------------------------------


def _raw_rows(x: torch.Tensor, width: int, name: str):
    """``x`` as ``[T, width]`` bf16 rows read in place (row stride a multiple of 4
    elements, 8-byte aligned); anything else is made contiguous first."""
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bf16")
    if x.shape[-1] != width:
        raise ValueError(f"{name} must have {width} channels per token, got {tuple(x.shape)}")
    try:
        x2 = x.view(-1, width)
    except RuntimeError:
        x2 = x.reshape(-1, width).contiguous()
    if x2.stride(1) != 1 or x2.stride(0) % 4 or x2.data_ptr() % 8 or (x2.shape[0] > 1 and x2.stride(0) < width):
        x2 = x2.contiguous()
    return x2, (x2.stride(0) if x2.shape[0] > 1 else width)


def _fused_update(q, k, v, decay, decay_bias, decay_scale_log, erase, write, num_heads, *, plan, scale, eps,
                  h0, ht, read_states, slots=None, n_slots=0):
    lib = _lib.load()
    _lib.require_gpu(q, k, v, decay, erase, write)
    H = num_heads
    K = k.shape[-1] // H
    V = v.shape[-1] // H
    rows = {}
    for name, t, wdt in (("q", q, H * K), ("k", k, H * K), ("v", v, H * V), ("decay", decay, H * K),
                         ("erase", erase, H * K), ("write", write, H * V)):
        rows[name] = _raw_rows(t, wdt, name)
    T = rows["k"][0].shape[0]
    if any(r[0].shape[0] != T for r in rows.values()) or plan.total_tokens != T:
        raise ValueError("projections and plan must cover the same tokens")
    bias, rate = _gate_params(decay_bias, decay_scale_log, H, K, k.device)
    x = _lib.Projections(
        q=rows["q"][0].data_ptr(), q_stride=rows["q"][1], k=rows["k"][0].data_ptr(), k_stride=rows["k"][1],
        v=rows["v"][0].data_ptr(), v_stride=rows["v"][1], decay=rows["decay"][0].data_ptr(),
        decay_stride=rows["decay"][1], erase=rows["erase"][0].data_ptr(), erase_stride=rows["erase"][1],
        write=rows["write"][0].data_ptr(), write_stride=rows["write"][1], decay_bias=bias.data_ptr(),
        decay_scale_log=rate.data_ptr(), eps=float(eps), reserved=0)
    dev = k.device
    q_hat = torch.empty(1, T, H, K, dtype=torch.bfloat16, device=dev)
    o = torch.empty(1, T, H, V, dtype=torch.bfloat16, device=dev)
    ws = _workspace(dev, workspace_bytes(plan.num_chunk, H, K, V, "snapshot", plan.num_sample))
    p = plan.abi()
    rs, s0, s1 = slots if slots is not None else (None, None, None)
    _lib.check(
        lib.memt_gdn2_chunk_update_fused(
            ctypes.addressof(x), q_hat.data_ptr(), _lib.ptr(h0), _lib.ptr(ht), _lib.ptr(read_states), n_slots,
            _lib.ptr(rs), _lib.ptr(s0), _lib.ptr(s1), o.data_ptr(), ctypes.byref(p), T, H, K, V, float(scale),
            _OUT["snapshot"], ws.data_ptr(), ws.numel(), _lib.stream_of(dev)),
        "chunk_update_fused",
    )
    return o


def token_memory_packed_fused(q, k, v, decay, decay_bias, decay_scale_log, erase, write, read_states, write_states, *,
                              lengths, scale, chunk_tokens, num_heads, eps: float = 1e-6):
    """The commit path of ``QwenMemoryBlock.packed`` (models/qwen/layer.py:132-150)
    from its raw projections: ``q, k, decay, erase`` ``[T, H*K]``, ``v, write``
    ``[T, H*V]`` bf16 (views of the projection outputs are read in place),
    ``decay_bias`` ``[H*K]``, ``decay_scale_log`` ``[H]``.  The gate and q/k
    prologue runs inside the update.  Returns ``(read [1,T,H,V] bf16,
    final [N,H,K,V] fp32)`` as ``token_memory_packed`` of the prologue's outputs."""
    if not lengths or any(int(n) <= 0 for n in lengths):
        raise ValueError("Packed sample lengths must be positive")
    H = num_heads
    K, V = k.shape[-1] // H, v.shape[-1] // H
    plan = packed_plan(lengths, k.device, chunk_tokens=chunk_tokens)
    expected = (plan.num_sample, H, K, V)
    for name, t in (("write_states", write_states), ("read_states", read_states)):
        if tuple(t.shape) != expected or t.dtype != torch.float32 or not t.is_cuda:
            raise ValueError(f"{name} must be fp32 {expected} on the GPU")
    h0, rs = _contig(write_states, read_states)
    final = torch.empty(expected, dtype=torch.float32, device=k.device)
    o = _fused_update(q, k, v, decay, decay_bias, decay_scale_log, erase, write, H, plan=plan, scale=scale, eps=eps,
                      h0=h0, ht=final, read_states=rs)
    return o, final


def token_memory_packed_fused_slots(q, k, v, decay, decay_bias, decay_scale_log, erase, write, pool, read_slots,
                                    write_slots, *, lengths, scale, chunk_tokens, num_heads, eps: float = 1e-6):
    """``token_memory_packed_fused`` on a state pool in place, as
    ``token_memory_packed_slots``.  Returns ``read``."""
    if not lengths or any(int(n) <= 0 for n in lengths):
        raise ValueError("Packed sample lengths must be positive")
    H = num_heads
    K, V = k.shape[-1] // H, v.shape[-1] // H
    pv = _pool_view(pool, H, K, V)
    plan = packed_plan(lengths, k.device, chunk_tokens=chunk_tokens)
    N = plan.num_sample
    rs = _slot_index(read_slots, N, pv.shape[0], k.device, "read_slots")
    ws_ = _slot_index(write_slots, N, pv.shape[0], k.device, "write_slots", distinct=True)
    return _fused_update(q, k, v, decay, decay_bias, decay_scale_log, erase, write, H, plan=plan, scale=scale,
                         eps=eps, h0=pv, ht=pv, read_states=pv, slots=(rs, ws_, ws_), n_slots=pv.shape[0])
