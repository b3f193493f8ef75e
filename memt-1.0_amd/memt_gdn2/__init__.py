"""MI355X (gfx950) GDN-2 native-memory hot path of MemT.

Drop-in operators for the memt_sglang memory plugin, backed by the
hand-written HIP library ``libmemt_gdn2.so`` (C ABI: include/memt_gdn2.h).
"""

from ._lib import LIB_PATH, load
from .layout import (
    WY_TILE_TOKENS,
    ChunkPlan,
    boundaries,
    build_chunk_plan,
    packed_plan,
    plan_from_cu_seqlens,
    validate_packed_inputs,
)
from .norm import MemTRMSNormGated
from .ops import (
    chunk_gdn2,
    chunk_gdn2_fwd_intra,
    chunk_local_cumsum,
    l2norm,
    l2norm_fwd,
    memt_gdn2_fwd_h,
    memt_gdn2_read_fwd,
    readout_decode,
    readout_fused,
    rms_norm_gated,
    snapshot_read,
    token_memory_packed,
    memory_prologue,
    read_slots,
    token_memory_packed_flash,
    token_memory_packed_fused,
    token_memory_packed_fused_slots,
    token_memory_packed_slots,
    workspace_bytes,
    write_gates,
)

RCP_LN2 = 1.4426950216  # FLA/ops/utils/constant.py:10

__all__ = [
    "LIB_PATH",
    "load",
    "RCP_LN2",
    "WY_TILE_TOKENS",
    "ChunkPlan",
    "boundaries",
    "build_chunk_plan",
    "packed_plan",
    "plan_from_cu_seqlens",
    "validate_packed_inputs",
    "MemTRMSNormGated",
    "chunk_gdn2",
    "chunk_gdn2_fwd_intra",
    "chunk_local_cumsum",
    "l2norm",
    "l2norm_fwd",
    "memt_gdn2_fwd_h",
    "memt_gdn2_read_fwd",
    "readout_fused",
    "readout_decode",
    "rms_norm_gated",
    "snapshot_read",
    "token_memory_packed",
    "token_memory_packed_flash",
    "workspace_bytes",
    "write_gates",
    "memory_prologue",
    "read_slots",
    "token_memory_packed_slots",
    "token_memory_packed_fused",
    "token_memory_packed_fused_slots",
]
