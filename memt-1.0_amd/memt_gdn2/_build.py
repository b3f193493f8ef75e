"""Build libmemt_gdn2.so for gfx950 from memt-1.0_amd/csrc with hipcc.

Run as ``python memt-1.0_amd/memt_gdn2/_build.py`` or call :func:`build`.
Objects go to ``memt-1.0_amd/_build/``; the shared library is written next
to this file so it is found in-tree.  The same call builds
``libmemt_roofs.so`` (the benchmark's read and MFMA roof probes, which the
package never loads).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
BUILD_DIR = ROOT / "_build"
LIB_NAME = "libmemt_gdn2.so"
LIB_PATH = PKG_DIR / LIB_NAME

SOURCES = ["abi.hip", "wy_kernel.hip", "state_kernel.hip", "scan_kernel.hip", "misc_kernels.hip", "prologue_kernel.hip", "plan.cpp"]
ROOFS_SOURCE = "roofs.hip"
ROOFS_PATH = PKG_DIR / "libmemt_roofs.so"

# -packed-fp32-ops off: hipcc must not emit packed fp32 VALU ops for this code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


# Per-source additions.  The column-split scan keeps its state in VALU-visible
# registers (it scales and converts the state every chunk), so its MFMA
# accumulators are allocated as VGPRs rather than AGPRs, which would need a copy
# each way per chunk.
EXTRA_FLAGS = {"scan_kernel.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the GDN-2 HIP library cannot be built")


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature: not an error.
    err = "\n".join(
        line for line in proc.stderr.splitlines() if "packed-fp32-ops" not in line and line.strip()
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile every source for gfx950 and link the shared library (always rebuilds)."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)])
    roofs_obj = BUILD_DIR / (Path(ROOFS_SOURCE).stem + ".o")
    cmds.append([hipcc, *HIPCC_FLAGS, "-c", str(CSRC / ROOFS_SOURCE), "-o", str(roofs_obj)])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for msg in ex.map(_run, cmds):
            if verbose and msg:
                print(msg, file=sys.stderr)
    for out, inputs in ((LIB_PATH, objs), (ROOFS_PATH, [roofs_obj])):
        tmp = out.with_suffix(".so.tmp")
        _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, inputs), "-o", str(tmp)])
        os.replace(tmp, out)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
