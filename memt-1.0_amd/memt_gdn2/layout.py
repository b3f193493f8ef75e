"""Write-event tiling and read-snapshot mapping of packed samples.

Mirrors the reference's plan types and builders
(models/qwen/ops/layout.py:18-135, models/qwen/ops/packed.py:16-31,
models/common/packed.py:8-34).  Plans are computed on the host from integer
boundaries by the library's C++ plan builder and uploaded with one
host-to-device copy; when the caller hands in host integers (``lengths``)
nothing is copied back from the device.
"""

from __future__ import annotations

import ctypes
from collections import OrderedDict
from dataclasses import dataclass
from itertools import accumulate

import numpy as np
import torch

from . import _lib

WY_TILE_TOKENS = 64  # models/common/constants.py:3

__all__ = [
    "WY_TILE_TOKENS",
    "ChunkPlan",
    "build_chunk_plan",
    "packed_plan",
    "plan_from_cu_seqlens",
    "boundaries",
    "validate_packed_inputs",
]

_CACHE_LIMIT = 8
_cache: "OrderedDict[tuple, ChunkPlan]" = OrderedDict()


@dataclass(frozen=True)
class ChunkPlan:
    """Write-event tiles, read snapshots and per-sample scan offsets.

    Field names and meanings follow the reference's ChunkPlan; every tensor
    is int32 on the plan's device.  ``table`` is the single device buffer the
    tensors view; :meth:`abi` describes it to the C ABI.
    """

    wy_tile_tokens: int
    num_event: int
    num_block: int
    num_sample: int
    num_chunk: int
    total_tokens: int
    event_slice: torch.Tensor
    chunk_indices: torch.Tensor
    sample_chunk_offsets: torch.Tensor
    chunk_block_ids: torch.Tensor
    chunk_is_block_start: torch.Tensor
    chunk_tok0: torch.Tensor
    chunk_len: torch.Tensor
    chunk_commits: torch.Tensor
    chunk_flags: torch.Tensor
    table: torch.Tensor

    def abi(self) -> _lib.Plan:
        return _lib.Plan(
            chunk_tok0=self.chunk_tok0.data_ptr(),
            chunk_len=self.chunk_len.data_ptr(),
            seq_chunk_offsets=self.sample_chunk_offsets.data_ptr(),
            chunk_block_ids=self.chunk_block_ids.data_ptr(),
            chunk_flags=self.chunk_flags.data_ptr(),
            n_chunk=self.num_chunk,
            n_seq=self.num_sample,
            n_block=self.num_block,
            reserved=0,
        )


def _host_ints(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().to("cpu", torch.int64).numpy()
    return np.asarray(x, dtype=np.int64).reshape(-1)


def _i32(x: np.ndarray) -> np.ndarray:
    if np.any(x < 0) or np.any(x > np.iinfo(np.int32).max):
        raise ValueError("token boundaries must fit int32")
    return np.ascontiguousarray(x, dtype=np.int32)


def _host_plan(read, sample, wy, event, commit_mask):
    """Integer chunk table of a set of boundaries, built by the library's host
    plan builder (memt_gdn2_plan_count / memt_gdn2_plan_build)."""
    if wy <= 0 or wy > WY_TILE_TOKENS:
        raise ValueError(f"wy_tile_tokens must be in 1..{WY_TILE_TOKENS}")
    if len(event) < 1 or event[0] != 0 or np.any(np.diff(event) < 0):
        raise ValueError("event boundaries must start at 0 and be non-decreasing")
    for name, arr in (("read", read), ("sample", sample)):
        if len(arr) < 1 or arr[0] != 0 or arr[-1] != event[-1] or np.any(np.diff(arr) < 0):
            raise ValueError(f"{name} boundaries must span the event tokens")
    n_event = len(event) - 1
    cm = None
    if commit_mask is not None:
        cm = np.ascontiguousarray(_host_ints(commit_mask).astype(bool), dtype=np.uint8)
        if len(cm) != n_event:
            raise ValueError("commit_mask needs one entry per write event")
    read, sample, event = _i32(read), _i32(sample), _i32(event)
    lib = _lib.load()
    n = ctypes.c_int32(0)
    _lib.check(lib.memt_gdn2_plan_count(event.ctypes.data, len(event), wy, ctypes.byref(n)), "build_chunk_plan")
    nc = n.value
    out = {name: np.zeros(nc, np.int32) for name in
           ("chunk_tok0", "chunk_len", "chunk_block_ids", "chunk_flags", "chunk_is_block_start", "chunk_commits")}
    out["chunk_indices"] = np.zeros(2 * nc, np.int32)
    out["sample_chunk_offsets"] = np.zeros(len(sample), np.int32)
    ptrs = {k: v.ctypes.data for k, v in out.items()}
    _lib.check(
        lib.memt_gdn2_plan_build(read.ctypes.data, len(read), sample.ctypes.data, len(sample), event.ctypes.data,
                                 len(event), None if cm is None else cm.ctypes.data, wy, nc, ptrs["chunk_tok0"],
                                 ptrs["chunk_len"], ptrs["sample_chunk_offsets"], ptrs["chunk_block_ids"],
                                 ptrs["chunk_flags"], ptrs["chunk_indices"], ptrs["chunk_is_block_start"],
                                 ptrs["chunk_commits"]),
        "build_chunk_plan",
    )
    return dict(num_event=n_event, num_block=len(read) - 1, num_sample=len(sample) - 1, num_chunk=nc,
                total_tokens=int(event[-1]), event_slice=event, **out)


_FIELDS = (
    "chunk_tok0",
    "chunk_len",
    "sample_chunk_offsets",
    "chunk_block_ids",
    "chunk_flags",
    "event_slice",
    "chunk_indices",
    "chunk_is_block_start",
    "chunk_commits",
)


def _upload(host: dict, wy: int, device) -> ChunkPlan:
    parts = [np.asarray(host[f], dtype=np.int32).reshape(-1) for f in _FIELDS]
    flat = np.concatenate(parts) if parts else np.zeros(0, np.int32)
    table = torch.from_numpy(flat).to(device=device)
    views = {}
    off = 0
    for name, p in zip(_FIELDS, parts):
        views[name] = table[off: off + len(p)]
        off += len(p)
    views["chunk_indices"] = views["chunk_indices"].view(-1, 2)
    return ChunkPlan(
        wy_tile_tokens=wy,
        num_event=host["num_event"],
        num_block=host["num_block"],
        num_sample=host["num_sample"],
        num_chunk=host["num_chunk"],
        total_tokens=host["total_tokens"],
        table=table,
        **views,
    )


def _cached(key, make):
    hit = _cache.get(key)
    if hit is not None:
        _cache.move_to_end(key)
        return hit
    plan = make()
    if len(_cache) >= _CACHE_LIMIT:
        _cache.popitem(last=False)
    _cache[key] = plan
    return plan


def _device_of(*xs, default=None):
    for x in xs:
        if isinstance(x, torch.Tensor):
            return x.device
    return torch.device(default if default is not None else "cuda")


def build_chunk_plan(turn_slice, sample_slice, wy_tile_tokens: int = WY_TILE_TOKENS, *, event_slice=None,
                     commit_mask=None, device=None) -> ChunkPlan:
    """Tile write events into <= ``wy_tile_tokens``-token chunks and map each
    chunk to its read snapshot (models/qwen/ops/layout.py:111-135).

    Boundaries may be device tensors (copied to the host, as the reference
    does) or host sequences.  Plans are cached by boundary values.
    """
    events = turn_slice if event_slice is None else event_slice
    dev = torch.device(device) if device is not None else _device_of(turn_slice, sample_slice, events)
    read = _host_ints(turn_slice)
    sample = _host_ints(sample_slice)
    event = _host_ints(events)
    cm = None if commit_mask is None else tuple(_host_ints(commit_mask).tolist())
    key = (tuple(read.tolist()), tuple(sample.tolist()), tuple(event.tolist()), cm, wy_tile_tokens, str(dev))
    return _cached(key, lambda: _upload(_host_plan(read, sample, wy_tile_tokens, event, cm), wy_tile_tokens, dev))


def boundaries(lengths, device) -> torch.Tensor:
    """``[0, l0, l0+l1, ...]`` as int32 (models/common/packed.py:8-9)."""
    return torch.tensor([0, *accumulate(lengths)], device=device, dtype=torch.int32)


def packed_plan(lengths, device, *, chunk_tokens: int) -> ChunkPlan:
    """Plan of a packed commit: every sample is cut into ``chunk_tokens``-token
    write events, all committed; each sample reads its own incoming state
    (models/qwen/ops/packed.py:16-31).  Built from host integers only."""
    lengths = [int(n) for n in lengths]
    if chunk_tokens <= 0:
        raise ValueError("chunk_tokens must be positive")
    samples = [0, *accumulate(lengths)]
    events = [0]
    offset = 0
    for n in lengths:
        events.extend(offset + t for t in range(chunk_tokens, n, chunk_tokens))
        offset += n
        events.append(offset)
    return build_chunk_plan(samples, samples, event_slice=events, commit_mask=[1] * (len(events) - 1),
                            device=device)


def plan_from_cu_seqlens(cu_seqlens, T: int, device, *, chunk_tokens=None, wy_tile_tokens: int = WY_TILE_TOKENS):
    """Plan of independent sequences (``cu_seqlens`` on the packed token axis,
    or one sequence of ``T`` tokens when None): each sequence starts from its
    own initial state; ``chunk_tokens`` optionally adds write-event cuts."""
    cu = [0, int(T)] if cu_seqlens is None else [int(x) for x in _host_ints(cu_seqlens)]
    lengths = [b - a for a, b in zip(cu[:-1], cu[1:])]
    if chunk_tokens is None:
        return build_chunk_plan(cu, cu, wy_tile_tokens, device=device)
    plan = packed_plan(lengths, device, chunk_tokens=chunk_tokens)
    if plan.wy_tile_tokens != wy_tile_tokens:
        raise ValueError("chunk_tokens plans use 64-token WY tiles")
    return plan


def validate_packed_inputs(block, hidden_states, read_states, write_states, lengths) -> None:
    """Metadata checks at the packed memory entry (models/common/packed.py:12-34)."""
    if (
        hidden_states.ndim != 2
        or hidden_states.shape[1] != block.hidden_size
        or not hidden_states.is_cuda
        or hidden_states.dtype != torch.bfloat16
    ):
        raise ValueError("Memory expects CUDA BF16 hidden states [tokens, hidden_size]")
    if not lengths or any(length <= 0 for length in lengths) or sum(lengths) != len(hidden_states):
        raise ValueError("Packed sample lengths must cover the hidden token rows")
    expected = (len(lengths), block.num_heads, block.head_dim, block.head_dim)
    if any(
        tuple(state.shape) != expected or state.dtype != torch.float32 or state.device != hidden_states.device
        for state in (read_states, write_states)
    ):
        raise ValueError(f"Memory expects FP32 states {expected} on the hidden device")
