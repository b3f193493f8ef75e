"""Chunk plans (models/qwen/ops/layout.py:47-135, models/qwen/ops/packed.py:16-31):
hand-counted tables, and the library's C++ plan builder against the
oracle's loop restatement.  CPU only (the builder is host code)."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import gdn2 as O

from memt_gdn2 import _lib
from memt_gdn2 import layout as L


def _host(plan, name):
    return getattr(plan, name).cpu().numpy().astype(np.int64)


def test_packed_plan_hand_counted():
    # samples [0,130,131,260]; 64-token events; every chunk fits one event
    plan = L.packed_plan([130, 1, 129], "cpu", chunk_tokens=64)
    assert plan.num_sample == 3 and plan.num_block == 3 and plan.num_event == 7 and plan.num_chunk == 7
    assert plan.total_tokens == 260
    assert list(_host(plan, "event_slice")) == [0, 64, 128, 130, 131, 195, 259, 260]
    assert list(_host(plan, "chunk_tok0")) == [0, 64, 128, 130, 131, 195, 259]
    assert list(_host(plan, "chunk_len")) == [64, 64, 2, 1, 64, 64, 1]
    assert list(_host(plan, "sample_chunk_offsets")) == [0, 3, 4, 7]
    assert list(_host(plan, "chunk_block_ids")) == [0, 0, 0, 1, 2, 2, 2]
    assert list(_host(plan, "chunk_is_block_start")) == [1, 0, 0, 1, 1, 0, 0]
    assert _host(plan, "chunk_indices").tolist() == [[e, 0] for e in range(7)]
    assert list(_host(plan, "chunk_flags")) == [3, 2, 2, 3, 3, 2, 2]


def test_sub_tiles_within_one_event():
    plan = L.build_chunk_plan([0, 40], [0, 40], 16, device="cpu")
    assert list(_host(plan, "chunk_tok0")) == [0, 16, 32]
    assert list(_host(plan, "chunk_len")) == [16, 16, 8]
    assert _host(plan, "chunk_indices").tolist() == [[0, 0], [0, 1], [0, 2]]


def test_read_blocks_differ_from_samples():
    # reads switch snapshot at token 50, mid-sample; commits off for event 1
    plan = L.build_chunk_plan([0, 50, 100], [0, 100], 16, event_slice=[0, 50, 100], commit_mask=[1, 0], device="cpu")
    assert list(_host(plan, "chunk_block_ids")) == [0, 0, 0, 0, 1, 1, 1, 1]
    assert list(_host(plan, "chunk_is_block_start")) == [1, 0, 0, 0, 1, 0, 0, 0]
    assert list(_host(plan, "chunk_commits")) == [1, 1, 1, 1, 0, 0, 0, 0]
    assert list(_host(plan, "sample_chunk_offsets")) == [0, 8]


@pytest.mark.parametrize("seed", range(6))
def test_vectorised_builder_matches_oracle_loops(seed):
    rng = np.random.default_rng(seed)
    lengths = [int(x) for x in rng.integers(1, 300, rng.integers(1, 6))]
    chunk_tokens = int(rng.choice([64, 100, 2048]))
    plan = L.packed_plan(lengths, "cpu", chunk_tokens=chunk_tokens)
    ref = O.packed_plan(lengths, chunk_tokens=chunk_tokens)
    for name in ("event_slice", "chunk_tok0", "chunk_len", "sample_chunk_offsets", "chunk_block_ids",
                 "chunk_is_block_start", "chunk_commits"):
        assert np.array_equal(_host(plan, name), getattr(ref, name)), name
    assert np.array_equal(_host(plan, "chunk_indices"), ref.chunk_indices)
    assert (plan.num_chunk, plan.num_event, plan.num_block, plan.num_sample) == (
        ref.num_chunk, ref.num_event, ref.num_block, ref.num_sample)


def test_plan_cache_by_value_and_single_upload():
    a = L.packed_plan([10, 20], "cpu", chunk_tokens=64)
    b = L.packed_plan([10, 20], "cpu", chunk_tokens=64)
    assert a is b
    # every field views the one uploaded table
    base = a.table.untyped_storage().data_ptr()
    for name in ("chunk_tok0", "chunk_len", "sample_chunk_offsets", "chunk_flags"):
        assert getattr(a, name).untyped_storage().data_ptr() == base


def test_boundaries_and_validation():
    assert L.boundaries([3, 4], "cpu").tolist() == [0, 3, 7]
    with pytest.raises(ValueError):
        L.build_chunk_plan([0, 5], [0, 6], device="cpu")
    with pytest.raises(ValueError):
        L.build_chunk_plan([0, 5], [0, 5], 128, device="cpu")

    class Block:
        hidden_size, num_heads, head_dim = 8, 2, 4

    h = torch.zeros(5, 8, dtype=torch.bfloat16)
    s = torch.zeros(1, 2, 4, 4)
    with pytest.raises(ValueError, match="CUDA BF16"):
        L.validate_packed_inputs(Block, h, s, s, [5])  # a CPU tensor is rejected like the reference


def _sorted_bounds(rng, total, n):
    """n - 1 interior boundaries in [0, total], repeats allowed (empty blocks / events)."""
    inner = np.sort(rng.integers(0, total + 1, n - 1)) if n > 1 else np.zeros(0, np.int64)
    return [0, *inner.tolist(), total]


@pytest.mark.parametrize("seed", range(20))
def test_builder_matches_oracle_on_independent_boundaries(seed):
    """Read, sample and event boundaries drawn independently (empty read blocks,
    empty events, samples that start mid-event), every WY tile size."""
    rng = np.random.default_rng(100 + seed)
    total = int(rng.integers(0, 700))
    read = _sorted_bounds(rng, total, int(rng.integers(1, 6)))
    sample = _sorted_bounds(rng, total, int(rng.integers(1, 6)))
    event = _sorted_bounds(rng, total, int(rng.integers(1, 9)))
    wy = int(rng.choice([1, 7, 16, 33, 64]))
    cm = [int(x) for x in rng.integers(0, 2, len(event) - 1)] if seed % 2 else None
    plan = L.build_chunk_plan(read, sample, wy, event_slice=event, commit_mask=cm, device="cpu")
    ref = O.build_chunk_plan(read, sample, wy, event_slice=event, commit_mask=cm)
    for name in ("event_slice", "chunk_tok0", "chunk_len", "sample_chunk_offsets", "chunk_block_ids",
                 "chunk_is_block_start", "chunk_commits"):
        assert np.array_equal(_host(plan, name), getattr(ref, name)), name
    assert np.array_equal(_host(plan, "chunk_indices").reshape(-1, 2), ref.chunk_indices.reshape(-1, 2))
    flags = ref.chunk_is_block_start * _lib.CHUNK_BLOCK_START + ref.chunk_commits * _lib.CHUNK_COMMIT
    assert np.array_equal(_host(plan, "chunk_flags"), flags)


def test_builder_c_abi_rejects_bad_boundaries():
    lib = _lib.load()
    i32 = lambda xs: (ctypes.c_int32 * len(xs))(*xs)  # noqa: E731
    n = ctypes.c_int32(-1)
    assert lib.memt_gdn2_plan_count(i32([0, 10, 5]), 3, 64, ctypes.byref(n)) == _lib.EINVAL  # decreasing
    assert lib.memt_gdn2_plan_count(i32([1, 10]), 2, 64, ctypes.byref(n)) == _lib.EINVAL  # not from 0
    assert lib.memt_gdn2_plan_count(i32([0, 10]), 2, 65, ctypes.byref(n)) == _lib.EINVAL  # tile > 64
    assert lib.memt_gdn2_plan_count(i32([0, 130]), 2, 64, ctypes.byref(n)) == _lib.OK and n.value == 3
    out = [(ctypes.c_int32 * 3)() for _ in range(4)]
    offs = (ctypes.c_int32 * 2)()
    ev = i32([0, 130])
    # chunk count that does not match the boundaries, and read boundaries that do not span the tokens
    assert lib.memt_gdn2_plan_build(ev, 2, ev, 2, ev, 2, None, 64, 2, out[0], out[1], offs, out[2], out[3],
                                    None, None, None) == _lib.EINVAL
    assert lib.memt_gdn2_plan_build(i32([0, 100]), 2, ev, 2, ev, 2, None, 64, 3, out[0], out[1], offs, out[2],
                                    out[3], None, None, None) == _lib.EINVAL
    assert lib.memt_gdn2_plan_build(ev, 2, ev, 2, ev, 2, None, 64, 3, out[0], out[1], offs, out[2], out[3],
                                    None, None, None) == _lib.OK
    assert list(out[0]) == [0, 64, 128] and list(out[1]) == [64, 64, 2] and list(offs) == [0, 3]
