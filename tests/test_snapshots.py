"""Memory snapshots on disk: the reference's memory-only safetensors v1 format
(runtime/snapshots.py:37-45,72-97: tensors ``memory.<layer>`` fp32 shaped like
a pool slot, metadata exactly {format: memt-memory-v1, identity}), round
trips, and every refusal, on a CPU fake pool."""

import os
import types

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from memt_gdn2.snapshots import SNAPSHOT_FORMAT, SnapshotDirectory, StateImage


def _pool(seed=0, slots=3):
    g = torch.Generator().manual_seed(seed)
    return types.SimpleNamespace(storage={0: torch.randn(slots, 1, 2, 4, 4, generator=g),
                                          5: torch.randn(slots, 1, 2, 4, 4, generator=g)})


def test_written_file_has_exactly_the_format(tmp_path):
    """The file read back with safetensors' own reader: exactly one fp32
    ``memory.<layer>`` tensor per layer, shaped like a slot, and exactly the
    two metadata entries."""
    src = _pool(1)
    rec = SnapshotDirectory(tmp_path).save(src, 1, "sess-1.safetensors", identity="nano@abc")
    assert rec.snapshot_id == "sess-1.safetensors" and rec.format == "memt-memory-v1" and rec.has_memory
    with safe_open(str(tmp_path / "sess-1.safetensors"), framework="pt") as f:
        assert f.metadata() == {"format": "memt-memory-v1", "identity": "nano@abc"}
        assert set(f.keys()) == {"memory.0", "memory.5"}
        for layer in (0, 5):
            t = f.get_tensor(f"memory.{layer}")
            assert t.dtype == torch.float32 and t.shape == (1, 2, 4, 4)
            assert torch.equal(t, src.storage[layer][1])
    assert sorted(os.listdir(tmp_path)) == ["sess-1.safetensors"]  # no temporary left behind


def test_round_trip_touches_only_the_target_slot(tmp_path):
    d = SnapshotDirectory(tmp_path)
    src, dst = _pool(1), _pool(2)
    d.save(src, 1, "s.safetensors", identity="x")
    before = {k: v.clone() for k, v in dst.storage.items()}
    rec = d.load(dst, 2, "s.safetensors", identity="x")
    assert rec.has_memory
    for layer in (0, 5):
        assert torch.equal(dst.storage[layer][2], src.storage[layer][1])
        assert torch.equal(dst.storage[layer][:2], before[layer][:2])


def test_file_written_by_the_format_alone_loads(tmp_path):
    """A file produced by any writer of the format (here safetensors directly)
    loads: the reader depends on the format, not on this module's writer."""
    meta = {"format": SNAPSHOT_FORMAT, "identity": "m"}
    st = {"memory.0": torch.full((1, 2, 4, 4), 0.5), "memory.5": torch.full((1, 2, 4, 4), -2.0)}
    save_file(st, str(tmp_path / "ext.safetensors"), metadata=meta)
    dst = _pool(3)
    SnapshotDirectory(tmp_path).load(dst, 0, "ext.safetensors", identity="m")
    assert torch.equal(dst.storage[0][0], st["memory.0"]) and torch.equal(dst.storage[5][0], st["memory.5"])


def test_without_memory_clears_the_slot(tmp_path):
    d = SnapshotDirectory(tmp_path)
    rec = d.save(_pool(1), 0, "empty.safetensors", identity="x", with_memory=False)
    assert not rec.has_memory
    with safe_open(str(tmp_path / "empty.safetensors"), framework="pt") as f:
        assert f.metadata() == {"format": "memt-memory-v1", "identity": "x"} and not list(f.keys())
    dst = _pool(3)
    assert d.load(dst, 1, "empty.safetensors", identity="x").has_memory is False
    assert not dst.storage[0][1].any() and not dst.storage[5][1].any()
    assert dst.storage[0][0].any()


def test_replace_rules(tmp_path):
    d = SnapshotDirectory(tmp_path)
    p = _pool(1)
    d.save(p, 0, "a.safetensors", identity="x")
    with pytest.raises(FileExistsError):
        d.save(p, 1, "a.safetensors", identity="x")
    q = _pool(4)
    d.load(q, 0, "a.safetensors", identity="x")
    assert torch.equal(q.storage[0][0], p.storage[0][0])  # the refused save left the file as it was
    d.save(p, 1, "a.safetensors", identity="x", replace=True)
    d.load(q, 0, "a.safetensors", identity="x")
    assert torch.equal(q.storage[0][0], p.storage[0][1])
    assert sorted(os.listdir(tmp_path)) == ["a.safetensors"]


@pytest.mark.parametrize("name", ["", ".hidden.safetensors", "a/b.safetensors", "x.pt", "a" * 121 + ".safetensors",
                                  None])
def test_bad_ids(tmp_path, name):
    with pytest.raises(ValueError):
        SnapshotDirectory(tmp_path).file_for(name)
    with pytest.raises(ValueError):
        SnapshotDirectory(None)
    assert SnapshotDirectory(tmp_path).file_for("a" * 120 + ".safetensors").name.startswith("a")


def test_symlink_target_refused(tmp_path):
    (tmp_path / "real.safetensors").write_bytes(b"")
    os.symlink(tmp_path / "real.safetensors", tmp_path / "link.safetensors")
    with pytest.raises(ValueError, match="symbolic link"):
        SnapshotDirectory(tmp_path).file_for("link.safetensors")


def test_load_refusals_leave_the_pool_unchanged(tmp_path):
    meta = {"format": "memt-memory-v1", "identity": "x"}
    good = {"memory.0": torch.zeros(1, 2, 4, 4), "memory.5": torch.zeros(1, 2, 4, 4)}
    cases = {
        "ident.safetensors": (good, {"format": "memt-memory-v1", "identity": "other"}),
        "fmt.safetensors": (good, {"format": "memt-memory-v0", "identity": "x"}),
        "extra_meta.safetensors": (good, {**meta, "note": "y"}),
        "layers.safetensors": ({"memory.0": torch.zeros(1, 2, 4, 4)}, meta),
        "dtype.safetensors": ({**good, "memory.5": torch.zeros(1, 2, 4, 4, dtype=torch.float64)}, meta),
        "shape.safetensors": ({**good, "memory.5": torch.zeros(2, 4, 4)}, meta),
        "nan.safetensors": ({**good, "memory.0": torch.full((1, 2, 4, 4), float("nan"))}, meta),
    }
    d = SnapshotDirectory(tmp_path)
    dst = _pool(5)
    before = {k: v.clone() for k, v in dst.storage.items()}
    for name, (tensors, md) in cases.items():
        save_file(tensors, str(tmp_path / name), metadata=md)
        with pytest.raises(ValueError):
            d.load(dst, 0, name, identity="x")
    (tmp_path / "junk.safetensors").write_bytes(b"not a safetensors file")
    with pytest.raises(ValueError):
        d.load(dst, 0, "junk.safetensors", identity="x")
    for layer in (0, 5):
        assert torch.equal(dst.storage[layer], before[layer])


def test_image_checks_before_writing():
    """restore() validates every layer before it writes any: a bad second layer
    leaves the first layer's slot untouched too."""
    pool = _pool(6)
    before = pool.storage[0].clone()
    img = StateImage("x", {0: torch.ones(1, 2, 4, 4), 5: torch.ones(1, 2, 5, 4)})
    with pytest.raises(ValueError):
        img.restore(pool, 0)
    assert torch.equal(pool.storage[0], before)
