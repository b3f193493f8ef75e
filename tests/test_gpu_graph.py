"""The update (two-level scan: WY, transition, combine and scan kernels), the
packed commit and the decode readout captured in one HIP graph: every replay,
with eager work on other memory between the replays, reproduces the eager
results bit for bit.  The library launches on the caller's stream and issues
no memset, copy or allocation of its own, so the whole path is capturable."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, to_dev

import memt_gdn2

pytestmark = pytest.mark.gpu


def test_path_replays_in_a_hip_graph(dev):
    print("hip graph replay", flush=True)
    T, H, D = 700, 2, 128  # 11 chunks on one sequence: groups of 4 chunks
    inp = O.synth_inputs(T, H, D, D, seed=70, h0_std=0.05)
    q, k, v, g = bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev)
    beta, h0 = to_dev(inp["beta"], dev), to_dev(inp["h0"], dev)
    lengths = [300, 400]
    rs = to_dev((np.random.default_rng(71).standard_normal((2, H, D, D)) * 0.05).astype(np.float32), dev)
    ws = rs.flip(0).contiguous()
    gen = torch.Generator(device=dev).manual_seed(72)
    S = torch.randn(8, H, D, D, generator=gen, device=dev) * 0.02
    qd = torch.nn.functional.normalize(torch.randn(8, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    gate = torch.randn(8, H, D, generator=gen, device=dev).to(torch.bfloat16)
    wn = (1 + 0.1 * torch.randn(D, generator=gen, device=dev)).to(torch.bfloat16)
    bb = beta.to(torch.bfloat16)

    def run():
        o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode="causal")
        read, final = memt_gdn2.token_memory_packed(q, k, v, g, bb, rs, ws, erase=None, lengths=lengths,
                                                    scale=D ** -0.5, chunk_tokens=256)
        out = memt_gdn2.readout_fused(S, qd, gate, wn, scale=D ** -0.5, eps=1e-6)
        return o, ht, read, final, out

    ref = [t.clone() for t in run()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    for i in range(4):
        junk = torch.randn(1 << 20, device=dev)  # eager work between replays
        assert bool(torch.isfinite(junk.sum()))
        for t in outs:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(("o", "ht", "read", "final", "readout"), outs, ref):
            assert torch.equal(got, want), (i, name)
