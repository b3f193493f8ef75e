"""The no-allocation chunked update (memt_gdn2_chunk_update_noalloc, static
device scratch) against memt_gdn2_chunk_update with a caller workspace, both
through the C ABI on the same inputs: bit-identical outputs and final states,
on two calls in a row, the second one smaller (the scratch keeps the first
call's contents), in causal and snapshot modes."""

import ctypes

import pytest
import torch

import memt_gdn2
from memt_gdn2 import _lib

pytestmark = pytest.mark.gpu


def _case(T, H, D, cu, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(1, T, H, D, generator=g, device=dev), dim=-1).to(torch.bfloat16)
    k = nrm(torch.randn(1, T, H, D, generator=g, device=dev), dim=-1).to(torch.bfloat16)
    v = torch.randn(1, T, H, D, generator=g, device=dev).to(torch.bfloat16)
    lg = torch.nn.functional.logsigmoid(torch.randn(1, T, H, D, generator=g, device=dev))
    beta = torch.sigmoid(torch.randn(1, T, H, D, generator=g, device=dev))
    h0 = torch.randn(len(cu) - 1, H, D, D, generator=g, device=dev) * 0.05
    rs = torch.randn(len(cu) - 1, H, D, D, generator=g, device=dev) * 0.05
    return q, k, v, lg, beta, h0, rs


def _call(lib, noalloc, args, plan, T, H, D, mode, dev):
    q, k, v, g, beta, h0, rs = args
    o = torch.full((1, T, H, D), float("nan"), dtype=torch.bfloat16, device=dev)
    ht = torch.full_like(h0, float("nan"))
    p = plan.abi()
    out_mode = _lib.OUT_CAUSAL if mode == "causal" else _lib.OUT_SNAPSHOT
    common = [q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), _lib.F32, None,
              h0.data_ptr(), ht.data_ptr(), rs.data_ptr() if mode == "snapshot" else None, None, o.data_ptr(),
              ctypes.byref(p), T, H, D, D, D ** -0.5, out_mode]
    stream = _lib.stream_of(dev)
    if noalloc:
        st = lib.memt_gdn2_chunk_update_noalloc(*common, stream)
    else:
        n = lib.memt_gdn2_chunk_update_workspace_size(plan.num_chunk, plan.num_sample, H, D, D, out_mode)
        ws = torch.empty(max(n, 256), dtype=torch.uint8, device=dev)
        st = lib.memt_gdn2_chunk_update(*common, ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, "chunk_update" + ("_noalloc" if noalloc else ""))
    torch.cuda.synchronize()
    return o, ht


@pytest.mark.parametrize("mode", ["causal", "snapshot"])
def test_noalloc_matches_workspace_entry(dev, mode):
    lib = memt_gdn2.load()
    H, D = 4, 128
    for T, cu, seed in ((3000, [0, 1100, 3000], 1), (300, [0, 300], 2)):  # the second call is smaller
        print(f"noalloc {mode} T={T} H={H} D={D} cu={cu}", flush=True)
        args = _case(T, H, D, cu, seed, dev)
        plan = memt_gdn2.plan_from_cu_seqlens(cu, T, dev)
        need = lib.memt_gdn2_chunk_update_workspace_size(plan.num_chunk, plan.num_sample, H, D, D,
                                                         _lib.OUT_CAUSAL)
        assert need <= _lib.NOALLOC_SCRATCH_BYTES
        o1, h1 = _call(lib, True, args, plan, T, H, D, mode, dev)
        o2, h2 = _call(lib, False, args, plan, T, H, D, mode, dev)
        assert torch.equal(o1, o2) and torch.equal(h1, h2)
        assert bool(torch.isfinite(h1).all()) and bool(torch.isfinite(o1.float()).all())
