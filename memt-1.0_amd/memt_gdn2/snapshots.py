"""Memory snapshots on disk: the fp32 state slots the update produces.

The file format is the reference's memory-only safetensors v1
(runtime/snapshots.py:34-104): one tensor ``memory.<layer>`` per memory layer,
shaped like a pool slot (``[1, H, K, V]`` fp32), and the metadata
``{"format": "memt-memory-v1", "identity": <model identity>}``.  A file written
here loads in the reference and back.  Writes go to a temporary file in the
target directory, are flushed to disk, and then replace (or, without
``overwrite``, hard-link to) the target, so a reader never sees a partial
snapshot.  Loading validates everything before it touches the slot.
"""

from __future__ import annotations

import os
import re
import tempfile
from pathlib import Path

import torch

SNAPSHOT_FORMAT = "memt-memory-v1"  # protocol/constants.py:4
MAX_SNAPSHOT_NAME_LENGTH = 120  # runtime/config.py:19

__all__ = ["SNAPSHOT_FORMAT", "snapshot_path", "save_memory", "load_memory", "save_snapshot", "load_snapshot"]

_NAME = re.compile(rf"[A-Za-z0-9_.-]{{1,{MAX_SNAPSHOT_NAME_LENGTH}}}\.safetensors")


def snapshot_path(directory, name) -> Path:
    """``directory/name`` for a plain ``*.safetensors`` name; no hidden files,
    no symlinked target (runtime/snapshots.py:14-31)."""
    if not directory or not isinstance(name, str) or not _NAME.fullmatch(name) or name.startswith("."):
        raise ValueError("Snapshot requires a configured directory and a simple .safetensors name")
    root = Path(directory).resolve()
    root.mkdir(parents=True, exist_ok=True)
    target = root / name
    if target.is_symlink():
        raise ValueError("Snapshot target must not be a symlink")
    return target


def _fsync_dir(path: Path) -> None:
    fd = os.open(path, os.O_RDONLY)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def save_memory(pool, slot: int, path: Path, *, identity: str, overwrite: bool = False, has_memory: bool = True):
    """Write slot ``slot`` of every layer of ``pool.storage`` to ``path``."""
    from safetensors.torch import save_file

    metadata = {"format": SNAPSHOT_FORMAT, "identity": identity}
    tensors = ({f"memory.{layer}": data[slot].detach().to("cpu").contiguous() for layer, data in pool.storage.items()}
               if has_memory else {})
    fd, tmp = tempfile.mkstemp(dir=path.parent, prefix=".memt-state-")
    os.close(fd)
    try:
        save_file(tensors, tmp, metadata=metadata)
        with open(tmp, "rb") as f:
            os.fsync(f.fileno())
        if overwrite:
            os.replace(tmp, path)
        else:
            os.link(tmp, path)  # fails if the target exists: never replace an existing key
        _fsync_dir(path.parent)
    finally:
        Path(tmp).unlink(missing_ok=True)
    return {"file": path.name, "format": SNAPSHOT_FORMAT, "has_memory": has_memory}


def load_memory(pool, slot: int, path: Path, *, identity: str) -> bool:
    """Validate ``path`` against the pool and copy it into slot ``slot`` (a
    snapshot without memory zeroes the slot).  Returns whether it held memory."""
    from safetensors import SafetensorError, safe_open

    try:
        with safe_open(path, framework="pt", device="cpu") as f:
            if f.metadata() != {"format": SNAPSHOT_FORMAT, "identity": identity}:
                raise ValueError("Snapshot model/encoding/format identity mismatch")
            names = {f"memory.{layer}": layer for layer in pool.storage}
            keys = set(f.keys())
            if keys and keys != names.keys():
                raise ValueError("Snapshot memory layer set mismatch")
            tensors = {layer: f.get_tensor(name) for name, layer in names.items()} if keys else {}
    except SafetensorError as error:
        raise ValueError("Invalid memory snapshot") from error
    for layer, t in tensors.items():
        if t.dtype != torch.float32 or t.shape != pool.storage[layer].shape[1:] or not bool(torch.isfinite(t).all()):
            raise ValueError("Snapshot requires finite FP32 tensors with exact layer shapes")
    for layer, storage in pool.storage.items():
        if tensors:
            storage[slot].copy_(tensors[layer])
        else:
            storage[slot].zero_()
    return bool(tensors)


def save_snapshot(pool, slot: int, snapshot_id: str, *, directory, identity: str, overwrite: bool = False,
                  has_memory: bool = True):
    """Persist a slot under a snapshot id (runtime/snapshots.py:106-119)."""
    path = snapshot_path(directory, snapshot_id)
    return {"snapshot_id": snapshot_id,
            **save_memory(pool, slot, path, identity=identity, overwrite=overwrite, has_memory=has_memory)}


def load_snapshot(pool, slot: int, snapshot_id: str, *, directory, identity: str):
    """Validate a snapshot and load it into a slot (runtime/snapshots.py:122-131)."""
    path = snapshot_path(directory, snapshot_id)
    has_memory = load_memory(pool, slot, path, identity=identity)
    return {"snapshot_id": snapshot_id, "file": snapshot_id, "format": SNAPSHOT_FORMAT, "has_memory": has_memory}
