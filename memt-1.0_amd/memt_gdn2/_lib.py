"""ctypes binding of libmemt_gdn2.so (the C ABI in include/memt_gdn2.h).

The library is loaded from this package directory.  There is no fallback:
if the library is missing or a tensor is not on a GPU, the call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmemt_gdn2.so"

OK = 0
EINVAL = -1
EUNSUPPORTED = -2
ELAUNCH = -3
EWORKSPACE = -4
ESCRATCH = -5
NOALLOC_SCRATCH_BYTES = 64 << 20

F32 = 0
BF16 = 1

GATE_SOFTCAP_SILU = 0
GATE_SIGMOID = 1

READOUT_L2NORM_Q = 1
READOUT_STATE_BF16 = 2

OUT_NONE = 0
OUT_SNAPSHOT = 1
OUT_CAUSAL = 2

CHUNK_BLOCK_START = 1
CHUNK_COMMIT = 2

ABI_VERSION = 7


class Plan(ctypes.Structure):
    """``memt_gdn2_plan``: device pointers of a chunk table."""

    _fields_ = [
        ("chunk_tok0", ctypes.c_void_p),
        ("chunk_len", ctypes.c_void_p),
        ("seq_chunk_offsets", ctypes.c_void_p),
        ("chunk_block_ids", ctypes.c_void_p),
        ("chunk_flags", ctypes.c_void_p),
        ("n_chunk", ctypes.c_int32),
        ("n_seq", ctypes.c_int32),
        ("n_block", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_PLAN = ctypes.POINTER(Plan)

# name -> (restype, argtypes)
_SIGNATURES = {
    "memt_gdn2_abi_version": (_I, []),
    "memt_gdn2_strerror": (ctypes.c_char_p, [_I]),
    "memt_gdn2_l2norm_fwd": (_I, [_P, _I, _P, _I, _P, _I64, _I, _F, _P]),
    "memt_gdn2_chunk_local_cumsum": (_I, [_P, _I, _P, _PLAN, _I, _I, _F, _I, _P]),
    "memt_gdn2_chunk_update_workspace_size": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "memt_gdn2_chunk_update": (
        _I,
        [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _PLAN, _I64, _I, _I, _I, _F, _I, _P, _SZ, _P],
    ),
    "memt_gdn2_chunk_update_noalloc": (
        _I,
        [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _PLAN, _I64, _I, _I, _I, _F, _I, _P],
    ),
    "memt_gdn2_chunk_update_fused": (
        _I,
        [ctypes.c_void_p, _P, _P, _P, _P, _I, _P, _P, _P, _P, _PLAN, _I64, _I, _I, _I, _F, _I, _P, _SZ, _P],
    ),
    "memt_gdn2_chunk_update_slots": (
        _I,
        [_P, _P, _P, _P, _P, _I, _P, _P, _I, _P, _P, _P, _P, _PLAN, _I64, _I, _I, _I, _F, _I, _P, _SZ, _P],
    ),
    "memt_gdn2_wy_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _PLAN, _I64, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "memt_gdn2_fwd_h": (_I, [_P, _P, _P, _P, _PLAN, _I64, _I, _I, _I, _P, _P, _P, _P, _SZ, _P]),
    "memt_gdn2_read_fwd": (_I, [_P, _P, _P, _PLAN, _I64, _I, _I, _I, _F, _P]),
    "memt_gdn2_read_fwd_slots": (_I, [_P, _P, _I, _P, _P, _PLAN, _I64, _I, _I, _I, _F, _P]),
    "memt_gdn2_rms_norm_gated": (_I, [_P, _P, _P, _P, _I64, _I, _F, _F, _I, _P]),
    "memt_gdn2_readout_fused": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _F, _I, _P]),
    "memt_gdn2_readout_decode": (
        _I, [_P, _P, _P, _I64, _P, _I64, _P, _P, _I, _I, _I, _I, _F, _F, _F, _F, _I, _I, _P]),
    "memt_gdn2_plan_count": (_I, [_P, _I, _I, _P]),
    "memt_gdn2_plan_build": (_I, [_P, _I, _P, _I, _P, _I, _P, _I, ctypes.c_int32, _P, _P, _P, _P, _P, _P, _P, _P]),
    "memt_gdn2_write_gates": (_I, [_P, _I64, _P, _P, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I, _I, _P]),
    "memt_gdn2_memory_prologue": (
        _I,
        [_P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _P, _I64, _P, _P, _P, _P, _I64, _I, _I, _F, _P],
    ),
}

class Projections(ctypes.Structure):
    """``memt_gdn2_projections``: raw projection rows of the memory block."""

    _fields_ = [
        ("q", ctypes.c_void_p), ("q_stride", ctypes.c_int64),
        ("k", ctypes.c_void_p), ("k_stride", ctypes.c_int64),
        ("v", ctypes.c_void_p), ("v_stride", ctypes.c_int64),
        ("decay", ctypes.c_void_p), ("decay_stride", ctypes.c_int64),
        ("erase", ctypes.c_void_p), ("erase_stride", ctypes.c_int64),
        ("write", ctypes.c_void_p), ("write_stride", ctypes.c_int64),
        ("decay_bias", ctypes.c_void_p),
        ("decay_scale_log", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python memt-1.0_amd/memt_gdn2/_build.py` "
            "(there is no CPU fallback for the GDN-2 memory path)"
        )
    lib = ctypes.CDLL(os.fspath(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.memt_gdn2_abi_version() != ABI_VERSION:
        raise RuntimeError("libmemt_gdn2.so ABI version mismatch; rebuild it")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    """Map a C-ABI status to the reference's exception types."""
    if status == OK:
        return
    msg = load().memt_gdn2_strerror(status).decode()
    if status == ELAUNCH:
        raise RuntimeError(f"{what}: {msg}")
    raise ValueError(f"{what}: {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor, or None."""
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    """Raw HIP stream handle of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("the GDN-2 memory kernels run on a GPU; got a CPU tensor")
