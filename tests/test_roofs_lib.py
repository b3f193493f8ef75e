"""The benchmark's roof-probe library (memt-1.0_amd/csrc/roofs.hip) loads,
exports its two probes and rejects bad arguments on the host (these calls
return before any GPU work).  The GDN-2 package never loads it."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


@pytest.fixture(scope="module")
def roofs():
    try:
        return bench._roofs_lib()
    except RuntimeError as e:
        pytest.fail(f"{e}: run __graft_entry__.build() first")


def test_probes_exported(roofs):
    assert hasattr(roofs, "memt_roofs_read") and hasattr(roofs, "memt_roofs_mfma")


def test_probes_reject_bad_arguments(roofs):
    assert roofs.memt_roofs_read(None, 1 << 20, None, 16, None) == -1
    assert roofs.memt_roofs_read(16, 1 << 20, None, 16, None) == -1      # no output buffer
    assert roofs.memt_roofs_read(16, 1 << 20, 16, 0, None) == -1         # no blocks
    assert roofs.memt_roofs_read(16, 1000, 16, 16, None) == -1           # not a multiple of 16 bytes
    assert roofs.memt_roofs_read(8, 1 << 20, 16, 16, None) == -1         # misaligned input
    assert roofs.memt_roofs_mfma(None, 16, 16, None) == -1
    assert roofs.memt_roofs_mfma(16, 0, 16, None) == -1
    assert roofs.memt_roofs_mfma(16, 16, 0, None) == -1


def test_package_does_not_load_the_probes():
    import memt_gdn2
    from memt_gdn2 import _lib

    memt_gdn2.load()
    assert "roofs" not in _lib.LIB_PATH.name
    text = " ".join(p.read_text() for p in (ROOT / "memt-1.0_amd" / "memt_gdn2").glob("*.py") if p.name != "_build.py")
    assert "libmemt_roofs" not in text
