"""The C-ABI library loads, exports every symbol include/memt_gdn2.h declares,
and rejects bad arguments on the host (these calls return before any GPU work)."""

import ctypes
import re
from pathlib import Path

import pytest

import memt_gdn2
from memt_gdn2 import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "memt_gdn2.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(memt_gdn2_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libmemt_gdn2.so is not built: run __graft_entry__.build() first")
    return memt_gdn2.load()


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib._SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version_and_strerror(lib):
    assert lib.memt_gdn2_abi_version() == _lib.ABI_VERSION
    assert int(re.search(r"#define MEMT_GDN2_ABI_VERSION (\d+)", HEADER.read_text()).group(1)) == _lib.ABI_VERSION
    for code in (0, -1, -2, -3, -4):
        assert lib.memt_gdn2_strerror(code)
    assert lib.memt_gdn2_strerror(-99) == b"unknown status"


def test_plan_struct_layout():
    # five pointers and four int32 in the header's order
    assert ctypes.sizeof(_lib.Plan) == 5 * 8 + 4 * 4
    assert [f[0] for f in _lib.Plan._fields_] == ["chunk_tok0", "chunk_len", "seq_chunk_offsets", "chunk_block_ids",
                                                  "chunk_flags", "n_chunk", "n_seq", "n_block", "reserved"]


def test_host_side_rejections(lib):
    plan = _lib.Plan(n_chunk=0, n_seq=1, n_block=1)
    # unsupported head dims
    assert lib.memt_gdn2_chunk_update(None, None, None, None, None, 0, None, None, None, None, None, None,
                                      ctypes.byref(plan), 0, 1, 96, 96, 1.0, 0, None, 0, None) == _lib.EUNSUPPORTED
    # a null plan
    assert lib.memt_gdn2_chunk_update(None, None, None, None, None, 0, None, None, None, None, None, None,
                                      None, 0, 1, 64, 64, 1.0, 0, None, 0, None) == _lib.EINVAL
    # bad out_mode / beta dtype
    assert lib.memt_gdn2_chunk_update(None, None, None, None, None, 0, None, None, None, None, None, None,
                                      ctypes.byref(plan), 0, 1, 64, 64, 1.0, 7, None, 0, None) == _lib.EINVAL
    assert lib.memt_gdn2_chunk_update(None, None, None, None, None, 5, None, None, None, None, None, None,
                                      ctypes.byref(plan), 0, 1, 64, 64, 1.0, 0, None, 0, None) == _lib.EUNSUPPORTED
    # missing workspace for a non-empty plan
    plan2 = _lib.Plan(chunk_tok0=16, chunk_len=16, seq_chunk_offsets=16, n_chunk=1, n_seq=1, n_block=1)
    ptr = 4096
    assert lib.memt_gdn2_chunk_update(None, ptr, ptr, ptr, ptr, 0, None, None, None, None, None, None,
                                      ctypes.byref(plan2), 64, 1, 64, 64, 1.0, 0, None, 0, None) == _lib.EWORKSPACE
    assert lib.memt_gdn2_l2norm_fwd(None, 1, None, 1, None, 4, 1024, 1e-6, None) == _lib.EINVAL
    assert lib.memt_gdn2_l2norm_fwd(ptr, 1, ptr, 1, None, 4, 1024, 1e-6, None) == _lib.EUNSUPPORTED
    assert lib.memt_gdn2_readout_fused(None, None, None, None, None, None, 1, 1, 128, 128, 1.0, 1e-6, 2.0, 0,
                                       None) == _lib.EINVAL
    assert lib.memt_gdn2_readout_fused(ptr, None, ptr, ptr, ptr, ptr, 1, 1, 128, 128, 1.0, 1e-6, 0.0, 0,
                                       None) == _lib.EINVAL  # soft cap must be positive
    assert lib.memt_gdn2_rms_norm_gated(ptr, ptr, ptr, ptr, 1, 64, 1e-6, 2.0, 9, None) == _lib.EINVAL
    ws = lib.memt_gdn2_chunk_update_workspace_size
    assert ws(128, 64, 16, 128, 128, 2) > ws(128, 64, 16, 128, 128, 1) > 0
    # one long sequence takes the two-level scan, whose group states (transition,
    # contribution and start state per group and head) add to the workspace
    extra = ws(128, 1, 16, 128, 128, 2) - ws(128, 64, 16, 128, 128, 2)
    assert extra >= 8 * 16 * 128 * 128 * 4 * 3


def test_d512_modes(lib):
    """d = 512 (the Flash head) takes the final-state and snapshot modes, also
    from raw projections; the causal output returns EUNSUPPORTED before any
    launch.  Its long sequences never take the two-level scan, so the
    workspace holds the chunk records only."""
    plan = _lib.Plan(n_chunk=0, n_seq=1, n_block=1)
    call = lambda mode: lib.memt_gdn2_chunk_update(  # noqa: E731
        None, None, None, None, None, 0, None, None, None, None, None, None, ctypes.byref(plan), 0, 1, 512, 512, 1.0,
        mode, None, 0, None)
    assert call(2) == _lib.EUNSUPPORTED
    assert call(7) == _lib.EINVAL
    x = _lib.Projections()
    assert lib.memt_gdn2_chunk_update_fused(ctypes.byref(x), None, None, None, None, 0, None, None, None, None,
                                            ctypes.byref(plan), 0, 1, 512, 512, 1.0, 2, None, 0,
                                            None) == _lib.EUNSUPPORTED
    ws = lib.memt_gdn2_chunk_update_workspace_size
    assert ws(256, 1, 2, 512, 512, 1) == ws(256, 64, 2, 512, 512, 1)
    assert ws(256, 1, 2, 256, 256, 1) > ws(256, 64, 2, 256, 256, 1)  # d = 256 does group


def test_python_layer_fails_loudly_without_gpu():
    import torch

    with pytest.raises(ValueError, match="GPU"):
        memt_gdn2.l2norm_fwd(torch.zeros(2, 64, dtype=torch.bfloat16))


def test_noalloc_rejects_problems_beyond_its_scratch(lib):
    """The no-allocation update checks its static scratch before touching the
    device: a plan needing more returns MEMT_GDN2_ESCRATCH (and the size
    function agrees with the scratch limit the header states)."""
    assert b"static scratch" in lib.memt_gdn2_strerror(_lib.ESCRATCH)
    dummy = (ctypes.c_int32 * 1)()
    n_chunk = 4096  # 4096 chunks x 16 heads at d=128: ~290 MiB of workspace
    plan = _lib.Plan(chunk_tok0=ctypes.addressof(dummy), chunk_len=ctypes.addressof(dummy),
                     seq_chunk_offsets=ctypes.addressof(dummy), chunk_block_ids=None, chunk_flags=None,
                     n_chunk=n_chunk, n_seq=1, n_block=1, reserved=0)
    need = lib.memt_gdn2_chunk_update_workspace_size(n_chunk, 1, 16, 128, 128, _lib.OUT_CAUSAL)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    st = lib.memt_gdn2_chunk_update_noalloc(None, None, None, None, None, _lib.F32, None, None, None, None, None,
                                            None, ctypes.byref(plan), 64 * n_chunk, 16, 128, 128, 0.088,
                                            _lib.OUT_CAUSAL, None)
    assert st == _lib.ESCRATCH
    assert lib.memt_gdn2_chunk_update_noalloc(None, None, None, None, None, _lib.F32, None, None, None, None, None,
                                              None, None, 0, 16, 128, 128, 0.088, _lib.OUT_CAUSAL,
                                              None) == _lib.EINVAL
