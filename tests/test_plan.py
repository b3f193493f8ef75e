"""Chunk plans (models/qwen/ops/layout.py:47-135, models/qwen/ops/packed.py:16-31):
hand-counted tables, and the product's vectorised builder against the
oracle's loop restatement.  CPU only."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O

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
