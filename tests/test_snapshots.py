"""Memory snapshots on disk (runtime/snapshots.py): the safetensors v1 format
with its metadata, round trips, and every refusal, on a CPU fake pool."""

import os
import types

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from memt_gdn2 import snapshots as S


def _pool(seed=0, slots=3):
    g = torch.Generator().manual_seed(seed)
    return types.SimpleNamespace(storage={0: torch.randn(slots, 1, 2, 4, 4, generator=g),
                                          5: torch.randn(slots, 1, 2, 4, 4, generator=g)})


def test_round_trip_and_format(tmp_path):
    src, dst = _pool(1), _pool(2)
    info = S.save_snapshot(src, 1, "sess-1.safetensors", directory=tmp_path, identity="nano@abc")
    assert info == {"snapshot_id": "sess-1.safetensors", "file": "sess-1.safetensors",
                    "format": "memt-memory-v1", "has_memory": True}
    with safe_open(tmp_path / "sess-1.safetensors", framework="pt") as f:
        assert f.metadata() == {"format": "memt-memory-v1", "identity": "nano@abc"}
        assert set(f.keys()) == {"memory.0", "memory.5"}
        assert f.get_tensor("memory.5").shape == (1, 2, 4, 4)
    before = {k: v.clone() for k, v in dst.storage.items()}
    out = S.load_snapshot(dst, 2, "sess-1.safetensors", directory=tmp_path, identity="nano@abc")
    assert out["has_memory"] is True
    for layer in (0, 5):
        assert torch.equal(dst.storage[layer][2], src.storage[layer][1])
        assert torch.equal(dst.storage[layer][:2], before[layer][:2])  # other slots untouched
    assert not [p for p in os.listdir(tmp_path) if p.startswith(".memt-state-")]  # no temporary left


def test_without_memory_zeroes_the_slot(tmp_path):
    S.save_snapshot(_pool(1), 0, "empty.safetensors", directory=tmp_path, identity="x", has_memory=False)
    dst = _pool(3)
    assert S.load_snapshot(dst, 1, "empty.safetensors", directory=tmp_path, identity="x")["has_memory"] is False
    assert not dst.storage[0][1].any() and not dst.storage[5][1].any()


def test_overwrite_rules(tmp_path):
    p = _pool(1)
    S.save_snapshot(p, 0, "a.safetensors", directory=tmp_path, identity="x")
    with pytest.raises(FileExistsError):
        S.save_snapshot(p, 1, "a.safetensors", directory=tmp_path, identity="x")
    S.save_snapshot(p, 1, "a.safetensors", directory=tmp_path, identity="x", overwrite=True)
    q = _pool(4)
    S.load_snapshot(q, 0, "a.safetensors", directory=tmp_path, identity="x")
    assert torch.equal(q.storage[0][0], p.storage[0][1])


@pytest.mark.parametrize("name", ["", ".hidden.safetensors", "a/b.safetensors", "x.pt", "a" * 121 + ".safetensors"])
def test_bad_names(tmp_path, name):
    with pytest.raises(ValueError):
        S.snapshot_path(tmp_path, name)
    with pytest.raises(ValueError):
        S.snapshot_path(None, "ok.safetensors")


def test_symlink_target_refused(tmp_path):
    (tmp_path / "real.safetensors").write_bytes(b"")
    os.symlink(tmp_path / "real.safetensors", tmp_path / "link.safetensors")
    with pytest.raises(ValueError, match="symlink"):
        S.snapshot_path(tmp_path, "link.safetensors")


def _write(path, tensors, meta):
    save_file(tensors, str(path), metadata=meta)


def test_load_refusals_leave_the_slot_unchanged(tmp_path):
    meta = {"format": "memt-memory-v1", "identity": "x"}
    good = {"memory.0": torch.zeros(1, 2, 4, 4), "memory.5": torch.zeros(1, 2, 4, 4)}
    cases = {
        "ident.safetensors": (good, {"format": "memt-memory-v1", "identity": "other"}),
        "fmt.safetensors": (good, {"format": "memt-memory-v0", "identity": "x"}),
        "layers.safetensors": ({"memory.0": torch.zeros(1, 2, 4, 4)}, meta),
        "dtype.safetensors": ({**good, "memory.5": torch.zeros(1, 2, 4, 4, dtype=torch.float64)}, meta),
        "shape.safetensors": ({**good, "memory.5": torch.zeros(2, 4, 4)}, meta),
        "nan.safetensors": ({**good, "memory.0": torch.full((1, 2, 4, 4), float("nan"))}, meta),
    }
    dst = _pool(5)
    before = {k: v.clone() for k, v in dst.storage.items()}
    for name, (tensors, md) in cases.items():
        _write(tmp_path / name, tensors, md)
        with pytest.raises(ValueError):
            S.load_snapshot(dst, 0, name, directory=tmp_path, identity="x")
    (tmp_path / "junk.safetensors").write_bytes(b"not a safetensors file")
    with pytest.raises(ValueError):
        S.load_snapshot(dst, 0, "junk.safetensors", directory=tmp_path, identity="x")
    for layer in (0, 5):
        assert torch.equal(dst.storage[layer], before[layer])
