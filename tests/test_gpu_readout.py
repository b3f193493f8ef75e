"""GPU parity of the decode readout, gated RMSNorm, l2norm and cumsum kernels
against the CPU oracle (same seeded inputs)."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, check, host, to_dev

import memt_gdn2

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _readout_inputs(B, H, K, V, seed):
    rng = np.random.default_rng(seed)
    S = (rng.standard_normal((B, H, K, V)) * 0.02).astype(np.float32)
    q = O.bf16_round(O.l2norm(rng.standard_normal((B, H, K)).astype(np.float32))[0])
    gate = O.bf16_round(rng.standard_normal((B, H, V)).astype(np.float32))
    w = O.bf16_round((1 + 0.1 * rng.standard_normal(V)).astype(np.float32))
    return S, q, gate, w


@pytest.mark.parametrize("gate_kind", ["softcap_silu", "sigmoid"])
@pytest.mark.parametrize("B,H,D", [(64, 16, 128), (3, 2, 64), (32, 4, 256)])
def test_readout_fused(dev, B, H, D, gate_kind):
    print(f"readout_fused B={B} H={H} D={D} gate={gate_kind}", flush=True)
    S, q, gate, w = _readout_inputs(B, H, D, D, seed=B * 31 + D)
    out = memt_gdn2.readout_fused(to_dev(S, dev), bf(q, dev), bf(gate, dev), bf(w, dev), scale=D ** -0.5,
                                  eps=1e-6, gate_kind=gate_kind)
    ref = O.readout_fused(S, q, gate, w, scale=D ** -0.5, eps=1e-6, gate_kind=gate_kind).reshape(B, H * D)
    check(f"readout B={B} H={H} D={D} {gate_kind}", host(out), ref, out_bf16=True)


def test_readout_slot_indexed(dev):
    B, H, D = 8, 4, 128
    S, q, gate, w = _readout_inputs(20, H, D, D, seed=5)
    slots = np.array([3, 19, 0, 7, 7, 12, 1, 5], dtype=np.int32)
    out = memt_gdn2.readout_fused(to_dev(S, dev), bf(q[:B], dev), bf(gate[:B], dev), bf(w, dev), scale=D ** -0.5,
                                  eps=1e-6, slot_idx=torch.from_numpy(slots))
    ref = O.readout_fused(S[slots], q[:B], gate[:B], w, scale=D ** -0.5, eps=1e-6).reshape(B, H * D)
    assert O.parity_err(host(out), ref, out_bf16=True) <= TOL


@pytest.mark.parametrize("gate_kind", ["softcap_silu", "sigmoid"])
def test_rms_norm_gated(dev, gate_kind):
    rng = np.random.default_rng(3)
    rows, dim = 300, 128
    x = O.bf16_round(rng.standard_normal((rows, dim)).astype(np.float32))
    g = O.bf16_round(rng.standard_normal((rows, dim)).astype(np.float32))
    w = O.bf16_round((1 + 0.1 * rng.standard_normal(dim)).astype(np.float32))
    out = memt_gdn2.rms_norm_gated(bf(x, dev), bf(g, dev), bf(w, dev), eps=1e-6, gate_kind=gate_kind)
    ref = O.rms_norm_gated(x, g, w, eps=1e-6, gate_kind=gate_kind)
    assert O.parity_err(host(out), ref, out_bf16=True) <= TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_l2norm(dev, dtype):
    rng = np.random.default_rng(4)
    x = O.bf16_round(rng.standard_normal((5, 37, 3, 128)).astype(np.float32))
    y, rstd = memt_gdn2.l2norm_fwd(to_dev(x, dev, dtype))
    y_ref, r_ref = O.l2norm(x, out_bf16=(dtype == torch.bfloat16))
    assert O.parity_err(host(y), y_ref, out_bf16=(dtype == torch.bfloat16)) <= TOL
    assert O.max_rel_err(host(rstd), r_ref) <= 1e-5


def test_chunk_local_cumsum(dev):
    rng = np.random.default_rng(6)
    T, H, S = 300, 3, 128
    g = (-np.logaddexp(0, -rng.standard_normal((1, T, H, S)))).astype(np.float32)
    cu = [0, 100, 163, 300]
    out = memt_gdn2.chunk_local_cumsum(to_dev(g, dev), 64, scale=O.RCP_LN2, cu_seqlens=cu)
    ref = O.chunk_local_cumsum(g, 64, scale=O.RCP_LN2, cu_seqlens=cu)
    assert O.max_rel_err(host(out), ref) <= 1e-5
    out_r = memt_gdn2.chunk_local_cumsum(to_dev(g, dev), 32, reverse=True)
    ref_r = np.zeros_like(ref)
    for c0 in range(0, T, 32):
        ref_r[:, c0:c0 + 32] = np.cumsum(g[:, c0:c0 + 32][:, ::-1], axis=1)[:, ::-1]
    assert O.max_rel_err(host(out_r), ref_r) <= 1e-5
