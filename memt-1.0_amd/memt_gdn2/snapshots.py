"""State snapshots on disk: the fp32 memory slots the update produces.

On-disk format.  It is the reference's memory-only safetensors v1, kept
identical so files move between the two implementations
(runtime/snapshots.py:37-45,72-97):

* one tensor ``memory.<layer>`` per memory layer, fp32, shaped like one pool
  slot (``[1, H, K, V]``);
* the metadata is exactly ``{"format": "memt-memory-v1", "identity": <model identity>}``;
* a file without tensors records "no memory", and loading it clears the slot.

Design.  A snapshot passes through an in-memory :class:`StateImage`: the host
copies of one slot's per-layer states plus the model identity.  Saving
captures the image, serialises it to a safetensors buffer and publishes the
buffer through a private temporary file in the target directory, so a reader
sees either the old file or the whole new one.  Loading decodes the file into
an image and checks all of it (format, identity, layer set, dtype, shape,
finiteness) before it writes a single element of the pool.  Every refusal is
a ``ValueError``; saving over an existing file without ``replace=True`` raises
``FileExistsError`` and leaves the file as it was.
"""

from __future__ import annotations

import os
import re
import secrets
from dataclasses import dataclass, field
from pathlib import Path

import torch

SNAPSHOT_FORMAT = "memt-memory-v1"  # the format tag of memory-only snapshot files
NAME_LIMIT = 120  # characters of a snapshot id before ".safetensors"
_ID = re.compile(r"[A-Za-z0-9_.-]{1,%d}\.safetensors" % NAME_LIMIT)
_PREFIX = "memory."

__all__ = ["SNAPSHOT_FORMAT", "StateImage", "SnapshotRecord", "SnapshotDirectory"]


def _tensor_name(layer) -> str:
    return f"{_PREFIX}{layer}"


@dataclass(frozen=True)
class StateImage:
    """One pool slot's memory states on the host, with the model identity.
    ``states`` maps each memory layer to its fp32 slot tensor; an empty map is
    a snapshot without memory."""

    identity: str
    states: dict = field(default_factory=dict)

    @property
    def has_memory(self) -> bool:
        return bool(self.states)

    @classmethod
    def capture(cls, pool, slot: int, identity: str, *, with_memory: bool = True) -> "StateImage":
        """Copy slot ``slot`` of every layer of ``pool.storage`` ({layer: [slots, ...]}) to the host."""
        if not with_memory:
            return cls(identity, {})
        return cls(identity, {layer: data[slot].detach().to("cpu", copy=True).contiguous()
                              for layer, data in pool.storage.items()})

    def encode(self) -> bytes:
        """The safetensors v1 bytes of this image."""
        from safetensors.torch import save

        return save({_tensor_name(layer): t for layer, t in self.states.items()},
                    metadata={"format": SNAPSHOT_FORMAT, "identity": self.identity})

    @classmethod
    def read(cls, path: Path, identity: str, layers) -> "StateImage":
        """Decode ``path`` for a pool with memory layers ``layers``; refuse a
        file of another format or identity, or with another layer set."""
        from safetensors import SafetensorError, safe_open

        wanted = {_tensor_name(layer): layer for layer in layers}
        try:
            with safe_open(str(path), framework="pt", device="cpu") as f:
                meta = f.metadata() or {}
                if meta != {"format": SNAPSHOT_FORMAT, "identity": identity}:
                    raise ValueError(f"snapshot {path.name} was written for format "
                                     f"{meta.get('format')!r} / identity {meta.get('identity')!r}, "
                                     f"not {SNAPSHOT_FORMAT!r} / {identity!r}")
                names = set(f.keys())
                if names and names != set(wanted):
                    raise ValueError(f"snapshot {path.name} holds layers {sorted(names)}, "
                                     f"the pool has {sorted(wanted)}")
                states = {wanted[n]: f.get_tensor(n) for n in names}
        except SafetensorError as err:
            raise ValueError(f"{path.name} is not a readable safetensors snapshot") from err
        return cls(identity, states)

    def check_against(self, pool) -> None:
        """Every state is finite fp32 with exactly the slot shape of its layer."""
        for layer, t in self.states.items():
            slot_shape = tuple(pool.storage[layer].shape[1:])
            if t.dtype != torch.float32 or tuple(t.shape) != slot_shape:
                raise ValueError(f"layer {layer}: snapshot tensor is {t.dtype} {tuple(t.shape)}, "
                                 f"the slot is torch.float32 {slot_shape}")
            if not bool(torch.isfinite(t).all()):
                raise ValueError(f"layer {layer}: snapshot tensor has non-finite values")

    def restore(self, pool, slot: int) -> None:
        """Write the image into ``slot`` of every layer (zeros when it has no
        memory); nothing is written unless the whole image fits the pool."""
        self.check_against(pool)
        for layer, data in pool.storage.items():
            if self.has_memory:
                data[slot].copy_(self.states[layer])
            else:
                data[slot].zero_()


@dataclass(frozen=True)
class SnapshotRecord:
    """What a save or load did: the snapshot id, its file, the format tag and
    whether the snapshot carries memory."""

    snapshot_id: str
    path: Path
    format: str
    has_memory: bool


class SnapshotDirectory:
    """Snapshots kept as ``<root>/<snapshot_id>``, ``snapshot_id`` a plain
    ``*.safetensors`` file name (letters, digits, ``_ . -``; not hidden)."""

    def __init__(self, root):
        if not root:
            raise ValueError("a snapshot directory must be configured")
        self.root = Path(root).resolve()

    def file_for(self, snapshot_id: str) -> Path:
        if not isinstance(snapshot_id, str) or snapshot_id.startswith(".") or not _ID.fullmatch(snapshot_id):
            raise ValueError(f"{snapshot_id!r} is not a plain <name>.safetensors snapshot id "
                             f"(at most {NAME_LIMIT} characters of [A-Za-z0-9_.-], not hidden)")
        self.root.mkdir(parents=True, exist_ok=True)
        target = self.root / snapshot_id
        if target.is_symlink():
            raise ValueError(f"{snapshot_id} is a symbolic link; snapshots are regular files")
        return target

    def save(self, pool, slot: int, snapshot_id: str, *, identity: str, replace: bool = False,
             with_memory: bool = True) -> SnapshotRecord:
        target = self.file_for(snapshot_id)
        image = StateImage.capture(pool, slot, identity, with_memory=with_memory)
        self._publish(target, image.encode(), replace)
        return SnapshotRecord(snapshot_id, target, SNAPSHOT_FORMAT, image.has_memory)

    def load(self, pool, slot: int, snapshot_id: str, *, identity: str) -> SnapshotRecord:
        target = self.file_for(snapshot_id)
        image = StateImage.read(target, identity, pool.storage.keys())
        image.restore(pool, slot)
        return SnapshotRecord(snapshot_id, target, SNAPSHOT_FORMAT, image.has_memory)

    def _publish(self, target: Path, payload: bytes, replace: bool) -> None:
        """Write ``payload`` to a private file beside ``target`` (exclusive
        create, flushed to disk), then move it onto ``target`` (``replace``) or
        hard-link it there (which fails if ``target`` exists), and flush the
        directory entry."""
        part = target.with_name(f".{target.name}.{os.getpid()}.{secrets.token_hex(6)}.part")
        fd = os.open(part, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
        try:
            with os.fdopen(fd, "wb") as out:
                out.write(payload)
                out.flush()
                os.fsync(out.fileno())
            if replace:
                os.replace(part, target)
            else:
                os.link(part, target)
        finally:
            part.unlink(missing_ok=True)
        dir_fd = os.open(target.parent, os.O_RDONLY)
        try:
            os.fsync(dir_fd)
        finally:
            os.close(dir_fd)
