"""GPU parity of the d = 128 / 256 / 512 snapshot reader (read_wide_kernel), the
reader of models/qwen/ops/read.py:10-39 and models/deepseek/ops/read.py:6-31:
every token reads bf16(scale * q . bf16(S_block)).

The kernel keeps a workgroup's state columns in registers for a run of
chunks, streams q through LDS in steps (half a chunk at d = 512), reloads the
state where the read block changes inside a run, and skips the empty second
half of a short chunk.  The cases below reach each of those: ragged samples
(chunks of 1, 63 and 65 tokens), read blocks that change inside one sample,
many heads over few tokens, and pool slots read in place.  Each compares with
the oracle's fp64 reader (one bf16 rounding of the output)."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, host, to_dev

import memt_gdn2

pytestmark = pytest.mark.gpu
TOL = 2e-3  # max|x - ref| / max|ref| (bf16 outputs: beyond one bf16 ulp of ref)


def _q(rng, T, H, D):
    return O.bf16_round(O.l2norm(rng.standard_normal((1, T, H, D)).astype(np.float32))[0])


@pytest.mark.parametrize("D", [128, 256, 512])
@pytest.mark.parametrize("H,lengths", [(3, [130, 1, 2000, 64, 63, 65]), (64, [40, 64, 1])])
def test_wide_reader_ragged_samples(dev, D, H, lengths):
    print(f"wide reader D={D} H={H} lengths={lengths}", flush=True)
    rng = np.random.default_rng(7 + D + H)
    T = sum(lengths)
    q = _q(rng, T, H, D)
    S = (rng.standard_normal((len(lengths), H, D, D)) * 0.05).astype(np.float32)
    out = memt_gdn2.snapshot_read(bf(q, dev), to_dev(S, dev), lengths, D ** -0.5, bf16_accumulator_output=True)
    ref = O.snapshot_read(q, S, lengths, D ** -0.5)
    assert O.parity_err(host(out), ref, out_bf16=True) <= TOL


@pytest.mark.parametrize("D", [128, 256, 512])
def test_wide_reader_block_changes_inside_a_run(dev, D):
    """Read blocks inside one sample: a workgroup's run of chunks crosses block
    boundaries (one of them a single token), and the state is reloaded there."""
    from memt_gdn2.layout import build_chunk_plan

    H, T = 4, 3000
    reads = [0, 100, 700, 701, 1500, 3000]
    print(f"wide reader D={D} read blocks {reads}", flush=True)
    rng = np.random.default_rng(11 + D)
    q = _q(rng, T, H, D)
    nb = len(reads) - 1
    S = (rng.standard_normal((nb, H, D, D)) * 0.05).astype(np.float32)
    plan = build_chunk_plan(reads, [0, T], device=dev)
    out = memt_gdn2.memt_gdn2_read_fwd(bf(q, dev), to_dev(S, dev), plan, D ** -0.5, out_dtype=torch.bfloat16)
    qh, sb = q[0].astype(np.float64), O.bf16_round(S).astype(np.float64)
    ref = np.zeros((T, H, D))
    for n in range(nb):
        a, b = reads[n], reads[n + 1]
        ref[a:b] = np.einsum("thk,hkv->thv", qh[a:b], sb[n]) * D ** -0.5
    assert O.parity_err(host(out)[0], ref, out_bf16=True) <= TOL


@pytest.mark.parametrize("D", [128, 256, 512])
def test_wide_reader_pool_slots(dev, D):
    """The pool read in place: sample n reads pool[slots[n]]."""
    H, lengths = 4, [1000, 5, 995]
    print(f"wide reader D={D} pool slots", flush=True)
    rng = np.random.default_rng(13 + D)
    q = _q(rng, sum(lengths), H, D)
    pool = (rng.standard_normal((7, H, D, D)) * 0.05).astype(np.float32)
    slots = np.array([5, 0, 3], dtype=np.int32)
    out = memt_gdn2.read_slots(bf(q, dev), to_dev(pool, dev), torch.tensor(slots, device=dev), lengths, D ** -0.5)
    ref = O.snapshot_read(q, pool[slots], lengths, D ** -0.5)
    assert O.parity_err(host(out), ref, out_bf16=True) <= TOL
