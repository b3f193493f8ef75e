"""Benchmark of the MI355X GDN-2 native-memory hot path.

Prints ONE JSON line.  The headline ``value`` is the chunked GDN-2 update
throughput (tokens/s) on the Nano-like single layer: B=1, H=16, T=8192,
dk=dv=128, 64-token chunks, bf16 q/k/v, fp32 g/beta, fp32 initial state,
causal chunk output (bf16) plus final state (fp32).  The same line carries
the decode readout (batch 64 sequences, H=16, d=128, fused RMSNorm + output
gate) in GB/s, the roofline of each, the roofs measured on the GPU (streaming
read, device copy, an MFMA loop and a library GEMM) and the CPU baseline
timed on the host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "memt-1.0_amd"))
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = "GDN-2 update tokens/s @H16 d128 T8K (%MFMA); decode readout GB/s (%HBM)"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 * 2 ** 20


def update_flops(T, H, K, V, C=64, causal=True):
    """Algorithmic flops of the update per (token, head): 6KV + 2CK + (C+1)V + C^2/3,
    plus (C+1)(K+V) for the causal output (triangles count their useful half)."""
    per = 6 * K * V + 2 * C * K + (C + 1) * V + C * C / 3
    if causal:
        per += (C + 1) * (K + V)
    return T * H * per


def update_bytes(T, H, K, V, N=1):
    """Algorithmic HBM bytes: q,k,v bf16, g,beta fp32, o bf16, h0 in and ht out fp32."""
    return T * H * (2 * (2 * K + V) + 4 * K + 4 * V + 2 * V) + N * H * K * V * 8


def readout_bytes(B, H, K, V):
    """fp32 state, bf16 q, gate and output, bf16 norm weight."""
    return B * H * (4 * K * V + 2 * K + 2 * V + 2 * V) + 2 * V


TRAFFIC_PROFILE = ROOT / "profiles" / "pmc_traffic_update_h16_t8192_d128_readout_b64.md"


def profiled_traffic():
    """HBM bytes per update step and per readout launch, from the committed
    FETCH_SIZE/WRITE_SIZE summary (two rocprofv3 --pmc passes over
    ``bench.py --calibrate``, scaled by the counters of a 1 GiB copy)."""
    out = {}
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            key, _, val = line.partition(":")
            if key in ("update_traffic_bytes_per_step", "readout_traffic_bytes_per_launch"):
                out[key] = int(val)
    except OSError:
        pass
    return out.get("update_traffic_bytes_per_step"), out.get("readout_traffic_bytes_per_launch")


def _inputs(T, H, K, V, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(1, T, H, K, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(1, T, H, K, generator=g), dim=-1)
    v = torch.randn(1, T, H, V, generator=g)
    lg = torch.nn.functional.logsigmoid(torch.randn(1, T, H, K, generator=g))
    beta = torch.sigmoid(torch.randn(1, T, H, V, generator=g))
    h0 = torch.randn(1, H, K, V, generator=g) * 0.02
    return dict(q=q.to(dev, torch.bfloat16), k=k.to(dev, torch.bfloat16), v=v.to(dev, torch.bfloat16),
                g=lg.to(dev), beta=beta.to(dev), h0=h0.to(dev))


def _inputs_on_device(T, H, K, V, seed, dev):
    """The same distributions as _inputs, drawn on the GPU (the wide-state sets are GBs)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(1, T, H, K, generator=g, device=dev), dim=-1).to(torch.bfloat16)
    k = nrm(torch.randn(1, T, H, K, generator=g, device=dev), dim=-1).to(torch.bfloat16)
    v = torch.randn(1, T, H, V, generator=g, device=dev).to(torch.bfloat16)
    lg = torch.nn.functional.logsigmoid(torch.randn(1, T, H, K, generator=g, device=dev))
    beta = torch.sigmoid(torch.randn(1, T, H, V, generator=g, device=dev))
    h0 = torch.randn(1, H, K, V, generator=g, device=dev) * 0.02
    return dict(q=q, k=k, v=v, g=lg, beta=beta, h0=h0)


def bench_update(dev, steps, warmup, T=8192, H=16, D=128, out_mode="causal", on_device=False):
    import memt_gdn2

    nbytes_set = update_bytes(T, H, D, D)
    nsets = max(4, int(np.ceil(2 * MALL_BYTES / nbytes_set)))
    make = _inputs_on_device if on_device else _inputs
    sets = [make(T, H, D, D, seed=20261201 + i, dev=dev) for i in range(nsets)]

    def step(i):
        s = sets[i % nsets]
        return memt_gdn2.chunk_gdn2(s["q"], s["k"], s["v"], s["g"], s["beta"], initial_state=s["h0"],
                                    out_mode=out_mode)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(steps):
        step(i)
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return dict(wall_s=wall, ms_per_step=wall * 1e3 / steps, event_ms_mean=sum(per) / steps,
                event_ms_median=statistics.median(per), nsets=nsets, set_bytes=nbytes_set)


def bench_readout(dev, steps, warmup, B=64, H=16, D=128, gate_kind="softcap_silu", passes=8):
    """Replay a captured graph of readouts over rotating state sets (> MALL).
    The graph holds `passes` rounds over the sets, so the host's gap between
    replays (about 8 us) is spread over that many more launches."""
    import memt_gdn2

    nb = readout_bytes(B, H, D, D)
    nsets = max(4, int(np.ceil(1.5 * MALL_BYTES / nb)))
    g = torch.Generator().manual_seed(20261203)
    sets = []
    for _ in range(nsets):
        S = (torch.randn(B, H, D, D, generator=g) * 0.02).to(dev)
        q = torch.nn.functional.normalize(torch.randn(B, H, D, generator=g), dim=-1).to(dev, torch.bfloat16)
        gate = torch.randn(B, H, D, generator=g).to(dev, torch.bfloat16)
        sets.append((S, q, gate))
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dev, torch.bfloat16)

    def run_all():
        for S, q, gate in sets:
            memt_gdn2.readout_fused(S, q, gate, w, scale=D ** -0.5, eps=1e-6, gate_kind=gate_kind)

    for _ in range(max(1, warmup)):
        run_all()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(passes):
            run_all()
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    reps = max(steps // 4, 10)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    launches = reps * passes * nsets
    ms = e0.elapsed_time(e1) / launches
    return dict(ms_per_launch=ms, gbs=nb / (ms * 1e-3) / 1e9, bytes=nb, nsets=nsets, launches=launches)


COPY_BYTES = 1 << 30  # calibration copy: reads and writes exactly this many bytes


def _event_ms(fn, reps, warmup=2):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def bench_prologue(dev, reps=20, T=8192, H=16, D=128):
    """The gate and q/k prologue of the memory block on raw projections, alone
    (HBM: 20 D bytes per token and head) and as part of the commit path,
    separate kernel vs folded into the update's WY kernel."""
    import memt_gdn2

    W = H * D
    g = torch.Generator(device=dev).manual_seed(20261206)
    qkv = torch.randn(T, 3 * W, generator=g, device=dev).to(torch.bfloat16)
    gates = torch.randn(T, 2 * W + D, generator=g, device=dev).to(torch.bfloat16)
    decay = torch.randn(T, W, generator=g, device=dev).to(torch.bfloat16)
    bias = (torch.randn(W, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    rate = (torch.randn(H, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    q, k, v = qkv[:, :W], qkv[:, W:2 * W], qkv[:, 2 * W:]
    erase, write = gates[:, :W], gates[:, W:2 * W]
    st = torch.randn(1, H, D, D, generator=g, device=dev) * 0.02
    pro_ms = _event_ms(lambda: memt_gdn2.memory_prologue(q, k, decay, bias, rate, erase, write, H), reps)
    pro_bytes = T * H * 20 * D

    def separate():
        qh, kt, beta, gg = memt_gdn2.memory_prologue(q, k, decay, bias, rate, erase, write, H)
        return memt_gdn2.token_memory_packed(qh, kt, v.reshape(1, T, H, D), gg, beta, st, st, erase=None,
                                             lengths=[T], scale=D ** -0.5, chunk_tokens=2048)

    def fused():
        return memt_gdn2.token_memory_packed_fused(q, k, v, decay, bias, rate, erase, write, st, st, lengths=[T],
                                                   scale=D ** -0.5, chunk_tokens=2048, num_heads=H)

    sep_ms = _event_ms(separate, reps)
    fus_ms = _event_ms(fused, reps)
    return {
        "workload": f"memory block commit from raw projections, T={T} H={H} d={D}, one sample, 2048-token events",
        "prologue_us": pro_ms * 1e3,
        "prologue_gbs": pro_bytes / (pro_ms * 1e-3) / 1e9,
        "prologue_hbm_frac": pro_bytes / (pro_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "prologue_algorithmic_bytes": pro_bytes,
        "commit_separate_prologue_ms": sep_ms,
        "commit_fused_prologue_ms": fus_ms,
    }


def bench_wide(dev, steps, warmup, T=16384, H=64, D=256, B=32, cpu=True):
    """The wide-state Flash-like shape: chunked update (causal) and a batch-B readout."""
    steps = min(steps, 20)
    up = bench_update(dev, steps, warmup, T, H, D, out_mode="causal", on_device=True)
    ro = bench_readout(dev, steps, warmup, B=B, H=H, D=D)
    ub, uf = update_bytes(T, H, D, D), update_flops(T, H, D, D, causal=True)
    t = up["event_ms_mean"] * 1e-3
    res = {
        "metric": "wide-state GDN-2 update tokens/s @H64 d256 T16K; decode readout GB/s @B32",
        "value": T / (up["ms_per_step"] * 1e-3), "unit": "tokens/s", "steps": steps, "warmup": warmup,
        "ms_per_step": up["ms_per_step"], "dtype": "bf16", "data": "synthetic (same distributions, drawn on the GPU)",
        "config": {"workload": f"chunked GDN-2 update, B=1 H={H} T={T} dk=dv={D} chunk=64, causal output + final state"},
        "roofline": {"bound": "hbm", "achieved": ub / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": ub / t / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": ub,
                     "mfma_frac": uf / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, "algorithmic_flops": uf},
        "readout": {"workload": f"decode readout B={B} H={H} dk=dv={D}", "value": ro["gbs"], "unit": "GB/s",
                    "us_per_launch": ro["ms_per_launch"] * 1e3, "frac": ro["gbs"] / HBM_PEAK_GBS},
    }
    if cpu:
        res["cpu_baseline"] = cpu_baseline_chunked(T, H, D, heads=4)
    return res


def bench_flash(dev, steps, warmup, T=8192, H=64, D=512, B=8, cpu=True):
    """The Flash model's memory shape (d=512, models/deepseek/ops/packed.py:70-108):
    a commit in snapshot mode (every token reads the incoming state, final
    state out) and a batch-B decode readout."""
    steps = min(steps, 10)
    up = bench_update(dev, steps, warmup, T, H, D, out_mode="snapshot", on_device=True)
    ro = bench_readout(dev, steps, warmup, B=B, H=H, D=D)
    ub, uf = update_bytes(T, H, D, D), update_flops(T, H, D, D, causal=False) + 2 * T * H * D * D
    t = up["event_ms_mean"] * 1e-3
    res = {
        "metric": "Flash-shape GDN-2 commit tokens/s @H64 d512 T8K; decode readout GB/s @B8",
        "value": T / (up["ms_per_step"] * 1e-3), "unit": "tokens/s", "steps": steps, "warmup": warmup,
        "ms_per_step": up["ms_per_step"], "dtype": "bf16", "data": "synthetic (same distributions, drawn on the GPU)",
        "config": {"workload": f"chunked GDN-2 commit, B=1 H={H} T={T} dk=dv={D} chunk=64, snapshot read + final state"},
        "roofline": {"bound": "hbm", "achieved": ub / t / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": ub / t / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": ub,
                     "mfma_frac": uf / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, "algorithmic_flops": uf},
        "readout": {"workload": f"decode readout B={B} H={H} dk=dv={D}", "value": ro["gbs"], "unit": "GB/s",
                    "us_per_launch": ro["ms_per_launch"] * 1e3, "frac": ro["gbs"] / HBM_PEAK_GBS},
    }
    if cpu:
        res["cpu_baseline"] = cpu_baseline_chunked(T, H, D, heads=2, out_mode="snapshot")
    return res


def segment_lengths(total=65536, n=4, seed=20261204):
    """The varlen workload's segment lengths: n draws from U[1024, 32768],
    rescaled to sum to `total` (rounded, the last one absorbing the rest)."""
    rng = np.random.default_rng(seed)
    raw = rng.uniform(1024, 32768, n)
    lengths = [int(round(x)) for x in raw * total / raw.sum()]
    lengths[-1] = total - sum(lengths[:-1])
    return lengths


def cpu_baseline_chunked(T, H, D, *, heads, runs=3, out_mode="causal", segments=None):
    """The PyTorch-CPU chunked port (oracle/gdn2_torch.py) on `heads` of the H
    heads (all T tokens), fp32, median of `runs`; the rate is scaled to all H
    heads (heads are independent and the port's cost is linear in them)."""
    from oracle.gdn2_torch import chunked_gdn2_torch

    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(20261207)
    q = torch.nn.functional.normalize(torch.randn(T, heads, D, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(T, heads, D, generator=g), dim=-1)
    v = torch.randn(T, heads, D, generator=g)
    lg = torch.nn.functional.logsigmoid(torch.randn(T, heads, D, generator=g))
    beta = torch.sigmoid(torch.randn(T, heads, D, generator=g))
    bounds = [0, T] if segments is None else [0, *np.cumsum(segments).tolist()]
    h0 = torch.randn(len(bounds) - 1, heads, D, D, generator=g) * 0.02
    chunked_gdn2_torch(q[:256], k[:256], v[:256], lg[:256], beta[:256], h0=h0[0], out_mode=out_mode)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for n in range(len(bounds) - 1):
            a, b = bounds[n], bounds[n + 1]
            chunked_gdn2_torch(q[a:b], k[a:b], v[a:b], lg[a:b], beta[a:b], h0=h0[n], out_mode=out_mode)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times) * H / heads
    return dict(value=T / t, unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"{heads} of the {H} heads over all {T} tokens (d={D}, {out_mode}), fp32 torch CPU, median of "
                       f"{runs} runs, scaled to {H} heads ({statistics.median(times):.2f} s per run)")


def bench_varlen(dev, steps, warmup, T=65536, H=16, D=128, cpu=True):
    """The varlen packed update: 4 segments (seeded lengths from U[1024, 32768]
    rescaled to 65536 tokens), per-segment initial states, causal output and
    per-segment final states."""
    import memt_gdn2

    lengths = segment_lengths(T)
    cu = [0, *np.cumsum(lengths).tolist()]
    N = len(lengths)
    sets = []
    for i in range(2):  # 2 x 1.9 GB of inputs: beyond the MALL
        s = _inputs_on_device(T, H, D, D, seed=20261204 + i, dev=dev)
        gen = torch.Generator(device=dev).manual_seed(20261214 + i)
        s["h0"] = torch.randn(N, H, D, D, generator=gen, device=dev) * 0.02
        sets.append(s)

    def step(i):
        s = sets[i % len(sets)]
        return memt_gdn2.chunk_gdn2(s["q"], s["k"], s["v"], s["g"], s["beta"], initial_state=s["h0"],
                                    cu_seqlens=cu, out_mode="causal")

    steps = min(steps, 30)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_time(e1) / steps
    ub, uf = update_bytes(T, H, D, D, N=N), update_flops(T, H, D, D, causal=True)
    out = {
        "metric": "varlen GDN-2 update tokens/s @4 segments, 65536 tokens, H16 d128",
        "value": T / (wall / steps), "unit": "tokens/s", "steps": steps, "warmup": warmup,
        "ms_per_step": wall * 1e3 / steps, "dtype": "bf16", "data": "synthetic (same distributions, drawn on the GPU)",
        "config": {"workload": f"varlen packed chunked GDN-2 update, segments {lengths} (cu_seqlens), H={H} "
                               f"dk=dv={D} chunk=64, per-segment initial states, causal output + final states"},
        "roofline": {"bound": "hbm", "achieved": ub / (ev_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": ub / (ev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "algorithmic_bytes": ub,
                     "event_ms_per_launch": ev_ms, "mfma_frac": uf / (ev_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
                     "algorithmic_flops": uf},
    }
    if cpu:
        out["cpu_baseline"] = cpu_baseline_chunked(T, H, D, heads=4, segments=lengths)
    return out


def bench_naive_recurrence_shape(dev, reps=200, T=512, H=4, D=64, cpu=True):
    """The naive-recurrence configuration (B=1 H=4 T=512 d=64, zero initial
    state): the GPU update per call, and the reference's CPU path, the
    token-by-token fp32 recurrence in torch (oracle/gdn2_torch.py)."""
    import memt_gdn2
    from oracle.gdn2_torch import recurrent_gdn2_torch

    s = _inputs(T, H, D, D, seed=20261201, dev=dev)
    h0 = torch.zeros(1, H, D, D, device=dev)
    ms = _event_ms(lambda: memt_gdn2.chunk_gdn2(s["q"], s["k"], s["v"], s["g"], s["beta"], initial_state=h0,
                                               out_mode="causal"), reps, warmup=10)
    out = {"workload": f"naive-recurrence configuration B=1 H={H} T={T} dk=dv={D}, zero initial state, causal "
                       f"output + final state",
           "gpu_us_per_call": ms * 1e3, "gpu_tokens_per_s": T / (ms * 1e-3)}
    if cpu:
        torch.set_num_threads(os.cpu_count() or 1)
        cpu_in = {n: s[n][0].float().cpu() for n in ("q", "k", "v", "g", "beta")}
        recurrent_gdn2_torch(*(cpu_in[n][:16] for n in ("q", "k", "v", "g", "beta")))
        times = []
        for _ in range(5):
            t0 = time.perf_counter()
            recurrent_gdn2_torch(*(cpu_in[n] for n in ("q", "k", "v", "g", "beta")))
            times.append(time.perf_counter() - t0)
        t = statistics.median(times)
        out["cpu_baseline"] = dict(value=T / t, unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                                   sample=f"the whole configuration, token loop in fp32 torch CPU, median of 5 runs "
                                          f"({t * 1e3:.1f} ms each)")
    return out


def bench_block_decode(dev, reps=50, B=64, H=16, D=128, hidden=2048):
    """The memory block's decode step (QwenMemoryBlock.packed, commit=False,
    B one-token samples): the q and output-gate projections (torch GEMMs)
    plus the fused readout kernel, on rotating read-state sets (beyond the
    MALL); and the fused readout kernel alone on the same sets."""
    import types

    import memt_gdn2
    from memt_gdn2.block import QwenMemoryBlock

    cfg = types.SimpleNamespace(hidden_size=hidden, num_heads=H, head_dim=D, chunk_tokens=2048, rms_norm_eps=1e-6,
                                output_gate_softcap=2.0)
    torch.manual_seed(20261208)
    block = QwenMemoryBlock(cfg, device=dev)
    with torch.no_grad():
        for name, p in block.named_parameters():
            p.copy_(torch.randn_like(p, dtype=torch.float32) * (p.shape[-1] ** -0.5 if p.ndim == 2 else 0.1))
    nb = readout_bytes(B, H, D, D)
    nsets = max(4, int(np.ceil(1.5 * MALL_BYTES / nb)))
    g = torch.Generator(device=dev).manual_seed(20261209)
    states = [torch.randn(B, H, D, D, generator=g, device=dev) * 0.02 for _ in range(nsets)]
    xs = [torch.randn(B, hidden, generator=g, device=dev).to(torch.bfloat16) for _ in range(nsets)]
    lengths = [1] * B
    i = [0]

    def step():
        j = i[0] % nsets
        i[0] += 1
        return block.packed(xs[j], states[j], lengths=lengths, commit=False, write_states=states[j])

    step_ms = _event_ms(step, reps, warmup=5)  # eager, host launch overhead included

    def graph_ms(fn, passes, reps_):
        """ms per call of fn() inside a captured graph of `passes` rounds over the sets."""
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(passes):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        return _event_ms(graph.replay, reps_, warmup=2) / (passes * nsets)

    def steps_all():
        for j in range(nsets):
            block.packed(xs[j], states[j], lengths=lengths, commit=False, write_states=states[j])

    step_graph_ms = graph_ms(steps_all, 2, 10)
    W = H * D
    qkvs = [torch.nn.functional.linear(x, block.in_proj.weight[:3 * W]) for x in xs]
    gates = [torch.randn(B, W, generator=g, device=dev).to(torch.bfloat16) for _ in range(nsets)]
    wn = block.o_norm.weight.to(torch.bfloat16)

    def kernels_all():
        for j in range(nsets):
            memt_gdn2.readout_decode(states[j], qkvs[j][:, :W], gates[j], wn, num_heads=H, scale=D ** -0.5, eps=1e-6)

    k_ms = graph_ms(kernels_all, 8, 20)
    return {"workload": f"memory block decode step, QwenMemoryBlock.packed(commit=False), B={B} one-token samples, "
                        f"H={H} d={D}, hidden {hidden}, {nsets} rotating read-state sets",
            "ms_per_step": step_ms, "ms_per_step_graph": step_graph_ms,
            "readout_kernel_us": k_ms * 1e3, "readout_kernel_gbs": nb / (k_ms * 1e-3) / 1e9,
            "readout_kernel_hbm_frac": nb / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "note": "ms_per_step is eager (host launch overhead included); ms_per_step_graph and the kernel time "
                    "come from captured graphs over the rotating sets"}


def _roofs_lib():
    """The benchmark's roof probes (memt-1.0_amd/csrc/roofs.hip), built beside the library."""
    import ctypes

    path = ROOT / "memt-1.0_amd" / "memt_gdn2" / "libmemt_roofs.so"
    if not path.exists():
        raise RuntimeError(f"{path} is missing: build it with `python memt-1.0_amd/memt_gdn2/_build.py`")
    lib = ctypes.CDLL(os.fspath(path))
    lib.memt_roofs_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.memt_roofs_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    return lib


MFMA_PROBE_CHAINS = 8        # independent MFMA chains per wave in roofs.hip
MFMA_PROBE_FLOP = 16 * 16 * 32 * 2  # one v_mfma_f32_16x16x32_bf16


def measured_roofs(dev, reps=20):
    """Roofs measured on this GPU, reported beside the spec peaks: a device
    copy of COPY_BYTES (reads and writes that many bytes), a streaming read of
    the same bytes and a dense bf16 MFMA loop (both hand-written probes), and
    a bf16 8192^3 GEMM through torch.mm (hipBLASLt)."""
    lib = _roofs_lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    x = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).normal_()
    y = torch.empty_like(x)
    copy_ms = _event_ms(lambda: y.copy_(x), reps, warmup=3)
    del y
    # the read probe over several grid sizes (grid-stride loops, four loads in
    # flight per thread); the fastest is the measured read rate
    read_grids = (1024, 2048, 4096, 8192, 16384)
    part = torch.empty(max(read_grids) * 256, dtype=torch.float32, device=dev)
    read_ms, read_blocks = None, None
    for g in read_grids:
        def read(g=g):
            if lib.memt_roofs_read(x.data_ptr(), COPY_BYTES, part.data_ptr(), g, stream) != 0:
                raise RuntimeError("read probe launch failed")

        ms = _event_ms(read, reps, warmup=3)
        if read_ms is None or ms < read_ms:
            read_ms, read_blocks = ms, g
    del x
    blocks = 2048
    iters = 2048
    acc = torch.empty(blocks * 256 * MFMA_PROBE_CHAINS * 4, dtype=torch.float32, device=dev)

    def mfma():
        if lib.memt_roofs_mfma(acc.data_ptr(), blocks, iters, stream) != 0:
            raise RuntimeError("MFMA probe launch failed")

    mfma_ms = _event_ms(mfma, reps, warmup=3)
    n = 8192
    a = torch.randn(n, n, device=dev).to(torch.bfloat16)
    b = torch.randn(n, n, device=dev).to(torch.bfloat16)
    c = torch.empty(n, n, device=dev, dtype=torch.bfloat16)
    gemm_ms = _event_ms(lambda: torch.mm(a, b, out=c), reps, warmup=3)
    del a, b, c, part, acc
    torch.cuda.empty_cache()
    copy_gbs = 2 * COPY_BYTES / (copy_ms * 1e-3) / 1e9
    read_gbs = COPY_BYTES / (read_ms * 1e-3) / 1e9
    mfma_tflops = blocks * 4 * MFMA_PROBE_CHAINS * iters * MFMA_PROBE_FLOP / (mfma_ms * 1e-3) / 1e12
    gemm_tflops = 2 * n ** 3 / (gemm_ms * 1e-3) / 1e12
    return {
        "streaming_read_probe_gbs": read_gbs,
        "streaming_read_probe_frac_of_spec": read_gbs / HBM_PEAK_GBS,
        "streaming_read_probe_workload": f"streaming read of {COPY_BYTES >> 30} GiB (16-byte non-temporal "
                                         f"loads), fastest of {len(read_grids)} grids ({read_blocks} x 256 "
                                         f"threads), mean of {reps}",
        "hbm_copy_gbs": copy_gbs,
        "hbm_copy_frac_of_spec": copy_gbs / HBM_PEAK_GBS,
        "hbm_copy_workload": f"torch device copy of {COPY_BYTES >> 30} GiB fp32 (read + write), mean of {reps}",
        "mfma_bf16_tflops": mfma_tflops,
        "mfma_bf16_frac_of_spec": mfma_tflops / MFMA_BF16_PEAK_TFLOPS,
        "mfma_bf16_workload": f"v_mfma_f32_16x16x32_bf16 loop, {MFMA_PROBE_CHAINS} chains x {iters} per wave, "
                              f"{blocks * 4} waves, every accumulator stored, mean of {reps}",
        "gemm_bf16_tflops": gemm_tflops,
        "gemm_bf16_frac_of_spec": gemm_tflops / MFMA_BF16_PEAK_TFLOPS,
        "gemm_bf16_workload": f"torch.mm bf16 {n}x{n}x{n} (hipBLASLt), mean of {reps}",
    }


def calibrate(dev, T=8192, H=16, D=128, reps=3):
    """Workload for hardware-counter runs (rocprofv3 --pmc): a device copy of
    COPY_BYTES (the reference for FETCH_SIZE / WRITE_SIZE per byte), then `reps`
    update steps and readouts on distinct inputs.  Prints the kernel inventory."""
    import memt_gdn2

    x = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).normal_()
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    sets = [_inputs(T, H, D, D, seed=20261201 + i, dev=dev) for i in range(reps)]
    for s in sets:
        memt_gdn2.chunk_gdn2(s["q"], s["k"], s["v"], s["g"], s["beta"], initial_state=s["h0"], out_mode="causal")
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(20261203)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dev, torch.bfloat16)
    for _ in range(reps):
        S = (torch.randn(64, H, D, D, generator=g) * 0.02).to(dev)
        q = torch.nn.functional.normalize(torch.randn(64, H, D, generator=g), dim=-1).to(dev, torch.bfloat16)
        gate = torch.randn(64, H, D, generator=g).to(dev, torch.bfloat16)
        memt_gdn2.readout_fused(S, q, gate, w, scale=D ** -0.5, eps=1e-6)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": COPY_BYTES, "update_steps": reps, "readouts": reps,
                      "update_algorithmic_bytes": update_bytes(T, H, D, D),
                      "readout_algorithmic_bytes": readout_bytes(64, H, D, D)}))


def cpu_baseline_update(T=8192, H=16, D=128, runs=5):
    """The PyTorch-CPU port (oracle/gdn2_torch.py) on the full workload, fp32."""
    from oracle.gdn2_torch import chunked_gdn2_torch

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(20261201)
    q = torch.nn.functional.normalize(torch.randn(T, H, D, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(T, H, D, generator=g), dim=-1)
    v = torch.randn(T, H, D, generator=g)
    lg = torch.nn.functional.logsigmoid(torch.randn(T, H, D, generator=g))
    beta = torch.sigmoid(torch.randn(T, H, D, generator=g))
    h0 = torch.randn(H, D, D, generator=g) * 0.02
    chunked_gdn2_torch(q[:512], k[:512], v[:512], lg[:512], beta[:512], h0=h0)  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        chunked_gdn2_torch(q, k, v, lg, beta, h0=h0, out_mode="causal")
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return dict(value=T / t, unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"full workload (T={T}, H={H}, d={D}, causal), fp32 torch CPU, median of {runs} runs "
                       f"({t:.2f} s each)")


def cpu_baseline_readout(B=64, H=16, D=128, runs=5):
    from oracle.gdn2_torch import readout_torch

    g = torch.Generator().manual_seed(20261203)
    S = torch.randn(B, H, D, D, generator=g) * 0.02
    q = torch.nn.functional.normalize(torch.randn(B, H, D, generator=g), dim=-1).to(torch.bfloat16)
    gate = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    readout_torch(S, q, gate, w, scale=D ** -0.5, eps=1e-6)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for _ in range(20):
            readout_torch(S, q, gate, w, scale=D ** -0.5, eps=1e-6)
        times.append((time.perf_counter() - t0) / 20)
    t = statistics.median(times)
    return dict(value=readout_bytes(B, H, D, D) / t / 1e9, unit="GB/s", cores=torch.get_num_threads(),
                kind="port", sample=f"B={B} H={H} d={D}, 20 launches x {runs} runs, median")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--mode", default="causal", choices=["causal", "snapshot"])
    ap.add_argument("--wide", action="store_true",
                    help="measure the wide-state workload instead (B=1 H=64 T=16384 d=256; batch-32 readout)")
    ap.add_argument("--flash", action="store_true",
                    help="measure the Flash memory shape instead (B=1 H=64 T=8192 d=512 commit; batch-8 readout)")
    ap.add_argument("--varlen", action="store_true",
                    help="measure the varlen packed update instead (4 segments, 65536 tokens, H=16 d=128)")
    ap.add_argument("--probes", action="store_true",
                    help="run only the measured roofs (read and MFMA probes, copy, GEMM), for counter runs")
    ap.add_argument("--calibrate", action="store_true",
                    help="run the hardware-counter workload (copy of known size, then update steps and readouts)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the GDN-2 memory path is built and measured on a single MI355X "
              "(heads and sequences shard across GPUs with no communication); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    import memt_gdn2

    memt_gdn2.load()
    dev = torch.device("cuda:0")
    T, H, D = 8192, 16, 128
    if args.calibrate:
        calibrate(dev, T, H, D)
        return
    if args.probes:
        print(json.dumps(measured_roofs(dev, reps=5)))
        return
    if args.wide:
        print(json.dumps(bench_wide(dev, args.steps, args.warmup, cpu=not args.no_cpu)))
        return
    if args.flash:
        print(json.dumps(bench_flash(dev, args.steps, args.warmup, cpu=not args.no_cpu)))
        return
    if args.varlen:
        print(json.dumps(bench_varlen(dev, args.steps, args.warmup, cpu=not args.no_cpu)))
        return

    roofs = measured_roofs(dev, reps=50)  # first: its 0.2 s of probes and GEMMs also brings the clocks up
    up = bench_update(dev, args.steps, args.warmup, T, H, D, out_mode=args.mode)
    snap = (bench_update(dev, max(10, args.steps // 2), args.warmup, T, H, D, out_mode="snapshot")
            if args.mode == "causal" else None)
    ro = bench_readout(dev, args.steps, args.warmup)
    pro = bench_prologue(dev)
    dec = bench_block_decode(dev)
    naive = bench_naive_recurrence_shape(dev, cpu=not args.no_cpu)

    causal = args.mode == "causal"
    up_traffic, ro_traffic = profiled_traffic()
    if not causal:
        up_traffic = None  # the committed counters cover the causal workload
    ub = update_bytes(T, H, D, D)
    uf = update_flops(T, H, D, D, causal=causal)
    t_up = up["event_ms_mean"] * 1e-3
    achieved = ub / t_up / 1e9
    result = {
        "metric": METRIC,
        "value": T / (up["ms_per_step"] * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": up["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded: q,k l2-normalised N(0,1), v N(0,1), g logsigmoid(N(0,1)), beta sigmoid(N(0,1)), h0 N(0,0.02^2))",
        "config": {
            "workload": f"chunked GDN-2 update, B=1 H={H} T={T} dk=dv={D} chunk=64, {args.mode} output + final state",
            "global_batch": 1,
            "seq_len": T,
            "heads": H,
            "head_dim": D,
            "parallelism": "single GPU",
            "input_sets_rotated": up["nsets"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "update step: wy_kernel, colscan_trans_kernel, combine_kernel and colscan_state_kernel, timed together per step",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": up_traffic,
            "traffic_source": TRAFFIC_PROFILE.name if up_traffic else None,
            "algorithmic_bytes": ub,
            "event_ms_per_launch": up["event_ms_mean"],
            "mfma_frac": uf / t_up / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "algorithmic_flops": uf,
        },
        "readout": {
            "workload": "decode readout B=64 H=16 dk=dv=128, fp32 state, fused RMSNorm + SoftCapSiLU gate, bf16 out",
            "value": ro["gbs"],
            "unit": "GB/s",
            "us_per_launch": ro["ms_per_launch"] * 1e3,
            "roofline": {"bound": "hbm", "achieved": ro["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": ro["gbs"] / HBM_PEAK_GBS, "traffic": ro_traffic, "algorithmic_bytes": ro["bytes"]},
            "state_sets_rotated": ro["nsets"],
        },
    }
    result["memory_block_commit"] = pro
    result["memory_block_decode"] = dec
    result["naive_recurrence_config"] = naive
    result["measured_roofs"] = roofs
    result["roofline"]["mfma_frac_of_measured"] = uf / t_up / 1e12 / roofs["mfma_bf16_tflops"]
    if snap is not None:
        result["snapshot_mode"] = {
            "workload": "token_memory_packed semantics (tokens read the incoming state), same shapes",
            "value": T / (snap["ms_per_step"] * 1e-3),
            "unit": "tokens/s",
            "ms_per_step": snap["ms_per_step"],
            "hbm_frac": update_bytes(T, H, D, D) / (snap["event_ms_mean"] * 1e-3) / 1e9 / HBM_PEAK_GBS,
        }
    if not args.no_cpu:
        cb = cpu_baseline_update(T, H, D)
        result["cpu_baseline"] = cb
        result["readout"]["cpu_baseline"] = cpu_baseline_readout()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
