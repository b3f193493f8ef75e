"""GPU parity of the chunked GDN-2 update (WY stage + state scan + outputs)
against the CPU oracle: the fp64 token recurrence on small cases, the fp64
chunked form (a different algorithm, pinned equal to the recurrence) on the
full-size workload's heads."""

import numpy as np
import pytest
import torch

from oracle import gdn2 as O
from gpu_util import bf, check, host, to_dev, workload_inputs

import memt_gdn2

pytestmark = pytest.mark.gpu
TOL = 2e-3  # max|x - ref| / max|ref| (bf16 outputs: beyond half a bf16 ulp of ref)


def _dev_inputs(inp, dev):
    return (bf(inp["q"], dev), bf(inp["k"], dev), bf(inp["v"], dev), to_dev(inp["g"], dev),
            to_dev(inp["beta"], dev), to_dev(inp["h0"], dev))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("T", [1, 63, 64, 200])
def test_causal_vs_recurrent(dev, T, D):
    print(f"causal T={T} D={D}", flush=True)
    H = 2
    inp = O.synth_inputs(T, H, D, D, seed=100 + T + D, h0_std=0.05)
    q, k, v, g, beta, h0 = _dev_inputs(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, out_mode="causal")
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], h0=inp["h0"])
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_varlen_bf16_beta_erase_events(dev):
    """Packed sequences, bf16 write gate, channel erase gate, write events."""
    rng = np.random.default_rng(9)
    T, H, D = 300, 3, 64
    cu = [0, 37, 37 + 130, T]
    inp = O.synth_inputs(T, H, D, D, seed=9, h0_std=0.1, n_seq=3)
    beta = O.bf16_round(inp["beta"])
    b = O.bf16_round(rng.uniform(0.3, 1.0, (1, T, H, D)).astype(np.float32))
    q, k, v, g, _, h0 = _dev_inputs(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, bf(beta, dev), b=bf(b, dev), initial_state=h0, cu_seqlens=cu,
                                 out_mode="causal", chunk_tokens=96)
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], beta, b=b, h0=inp["h0"],
                                    cu_seqlens=cu)
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL


def test_token_memory_packed(dev):
    """The plugin drop-in: commits from write_states, reads read_states."""
    T, H, D = 260, 2, 128
    lengths = [130, 1, 129]
    inp = O.synth_inputs(T, H, D, D, seed=21, h0_std=0.05, n_seq=3)
    rs = (np.random.default_rng(22).standard_normal((3, H, D, D)) * 0.05).astype(np.float32)
    q, k, v, g, _, ws = _dev_inputs(inp, dev)
    beta = O.bf16_round(inp["beta"])
    read, final = memt_gdn2.token_memory_packed(q, k, v, g, bf(beta, dev), to_dev(rs, dev), ws, erase=None,
                                                lengths=lengths, scale=D ** -0.5, chunk_tokens=64)
    r_ref, f_ref = O.token_memory_packed(inp["q"], inp["k"], inp["v"], inp["g"], beta, rs, inp["h0"], erase=None,
                                         lengths=lengths, scale=D ** -0.5, chunk_tokens=64)
    assert O.max_rel_err(host(final), f_ref) <= TOL
    assert O.parity_err(host(read), r_ref, out_bf16=True) <= TOL


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("lengths", [[130, 1, 129], [5000, 3, 2300], [64]])
def test_snapshot_read_in_scan_equals_reader(dev, D, lengths):
    """At d <= 128 the snapshot-mode read runs inside the scan kernel; its
    output must be the standalone reader's bit for bit (same operand rounding,
    slot order and step order), on the plain and the two-level scan, and the
    oracle's within the tolerance."""
    print(f"fused snapshot read D={D} lengths={lengths}", flush=True)
    H, N = 2, len(lengths)
    T = sum(lengths)
    inp = O.synth_inputs(T, H, D, D, seed=41 + D + T, h0_std=0.05, n_seq=N)
    rs = (np.random.default_rng(42 + T).standard_normal((N, H, D, D)) * 0.05).astype(np.float32)
    q, k, v, g, _, ws = _dev_inputs(inp, dev)
    beta = O.bf16_round(inp["beta"])
    rs_d = to_dev(rs, dev)
    read, final = memt_gdn2.token_memory_packed(q, k, v, g, bf(beta, dev), rs_d, ws, erase=None,
                                                lengths=lengths, scale=D ** -0.5, chunk_tokens=2048)
    alone = memt_gdn2.snapshot_read(q, rs_d, lengths, D ** -0.5, bf16_accumulator_output=True)
    torch.cuda.synchronize()
    assert torch.equal(read, alone)
    r_ref = O.snapshot_read(inp["q"], rs, lengths, D ** -0.5)
    assert O.parity_err(host(read), r_ref, out_bf16=True) <= TOL


@pytest.mark.parametrize("D", [64, 128])
def test_snapshot_read_in_scan_with_read_blocks_inside_a_sample(dev, D):
    """Read boundaries inside a sample (turns): the scan's read changes its
    state where the read block changes, on the plain and the two-level scan;
    bit for bit the standalone reader's output on the same plan."""
    from memt_gdn2.layout import build_chunk_plan
    from memt_gdn2.ops import _chunk_update

    H = 2
    for T, reads in ((400, [0, 70, 130, 131, 400]), (6000, [0, 700, 1900, 4100, 6000])):
        print(f"read blocks inside a sample D={D} T={T} reads={reads}", flush=True)
        inp = O.synth_inputs(T, H, D, D, seed=51 + T + D, h0_std=0.05)
        nb = len(reads) - 1
        rs = (np.random.default_rng(52 + T).standard_normal((nb, H, D, D)) * 0.05).astype(np.float32)
        q, k, v, g, _, h0 = _dev_inputs(inp, dev)
        beta = bf(O.bf16_round(inp["beta"]), dev)
        rs_d = to_dev(rs, dev)
        plan = build_chunk_plan(reads, [0, T], device=q.device)
        o, ht = _chunk_update(q, k, v, g, beta, None, h0, rs_d, plan, D ** -0.5, "snapshot")
        alone = memt_gdn2.memt_gdn2_read_fwd(q, rs_d, plan, D ** -0.5, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.equal(o, alone.view_as(o))
        qh, sb = host(q)[0].astype(np.float64), O.bf16_round(rs).astype(np.float64)
        ref = np.zeros((T, H, D))
        for n in range(nb):
            a, b = reads[n], reads[n + 1]
            ref[a:b] = np.einsum("thk,hkv->thv", qh[a:b], sb[n]) * D ** -0.5
        assert O.parity_err(host(o)[0], ref, out_bf16=True) <= TOL
        _, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], O.bf16_round(inp["beta"]),
                                    h0=inp["h0"])
        assert O.max_rel_err(host(ht), h_ref) <= TOL


def test_snapshot_read_in_scan_past_the_plan_cache(dev):
    """16 sequences x 16 heads fill the launch, so the plain scan runs and each
    workgroup walks 66 chunks: the read's q rows for chunk 64 come from the plan
    tables directly rather than the scan's 64-chunk cache.  Bit for bit the
    standalone reader."""
    H, D, N, n = 16, 64, 16, 4200
    T = N * n
    print(f"fused snapshot read past the plan cache T={T} H={H} D={D}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(61)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(1, T, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    k = nrm(torch.randn(1, T, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    v = torch.randn(1, T, H, D, generator=gen, device=dev).to(torch.bfloat16)
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, H, D, generator=gen, device=dev))
    beta = torch.sigmoid(torch.randn(1, T, H, D, generator=gen, device=dev))
    rs = torch.randn(N, H, D, D, generator=gen, device=dev) * 0.05
    ws = torch.randn(N, H, D, D, generator=gen, device=dev) * 0.05
    read, final = memt_gdn2.token_memory_packed(q, k, v, g, beta, rs, ws, erase=None, lengths=[n] * N,
                                                scale=D ** -0.5, chunk_tokens=2048)
    alone = memt_gdn2.snapshot_read(q, rs, [n] * N, D ** -0.5, bf16_accumulator_output=True)
    torch.cuda.synchronize()
    assert torch.equal(read, alone)
    assert bool(torch.isfinite(final).all())


@pytest.mark.parametrize("T", [300, 6000])
def test_snapshot_read_with_final_states_over_the_read_states(dev, T):
    """memt_gdn2_chunk_update with ht naming the read states' memory: the read
    must see the states from before the update (it then runs as its own pass,
    not inside the scan), on the plain and the two-level scan."""
    import ctypes
    from memt_gdn2 import _lib
    from memt_gdn2.layout import packed_plan
    from memt_gdn2.ops import _DT, _OUT, _workspace, workspace_bytes

    H, D = 2, 128
    print(f"final states over the read states T={T}", flush=True)
    inp = O.synth_inputs(T, H, D, D, seed=71 + T, h0_std=0.05)
    q, k, v, g, _, h0 = _dev_inputs(inp, dev)
    beta = bf(O.bf16_round(inp["beta"]), dev)
    rs = torch.randn(1, H, D, D, generator=torch.Generator(device=dev).manual_seed(72), device=dev) * 0.05
    before = rs.clone()
    plan = packed_plan([T], dev, chunk_tokens=2048)
    o = torch.empty(1, T, H, D, dtype=torch.bfloat16, device=dev)
    ws = _workspace(dev, workspace_bytes(plan.num_chunk, H, D, D, "snapshot", plan.num_sample))
    p = plan.abi()
    lib = _lib.load()
    _lib.check(lib.memt_gdn2_chunk_update(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), _DT[beta.dtype], None,
        h0.data_ptr(), rs.data_ptr(), rs.data_ptr(), None, o.data_ptr(), ctypes.byref(p), T, H, D, D,
        float(D ** -0.5), _OUT["snapshot"], ws.data_ptr(), ws.numel(), _lib.stream_of(dev)), "chunk_update")
    alone = memt_gdn2.snapshot_read(q, before, [T], D ** -0.5, bf16_accumulator_output=True)
    torch.cuda.synchronize()
    assert torch.equal(o, alone)
    _, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], O.bf16_round(inp["beta"]), h0=inp["h0"])
    assert O.max_rel_err(host(rs), h_ref) <= TOL


def test_snapshot_mode_and_no_initial_state(dev):
    T, H, D = 100, 2, 64
    inp = O.synth_inputs(T, H, D, D, seed=31)
    q, k, v, g, beta, _ = _dev_inputs(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, out_mode="snapshot")
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], out_mode="snapshot")
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert np.all(host(o) == 0.0) and np.all(o_ref == 0.0)
    o2, ht2 = memt_gdn2.chunk_gdn2(q, k, v, g, beta, out_mode="none")
    assert o2 is None and torch.equal(ht2, ht)


def test_wy_stage_reference_layout(dev):
    """chunk_gdn2_fwd_intra outputs vs the oracle's per-chunk WY quantities."""
    T, H, D = 150, 2, 64
    inp = O.synth_inputs(T, H, D, D, seed=41)
    gk = O.chunk_local_cumsum(inp["g"], 64, scale=O.RCP_LN2).astype(np.float32)
    q, k, v, _, beta, _ = _dev_inputs(inp, dev)
    scale = D ** -0.5
    w, u, qg, kg, Aqk, Akk = memt_gdn2.chunk_gdn2_fwd_intra(q, k, v, to_dev(gk, dev), None, beta, scale,
                                                            disable_recompute=True)
    w, u, qg, kg, Aqk, Akk = (host(x) for x in (w, u, qg, kg, Aqk, Akk))
    for h in range(H):
        for c0 in range(0, T, 64):
            c1 = min(c0 + 64, T)
            n = c1 - c0
            wy = O.wy_chunk(inp["k"][0, c0:c1, h], inp["v"][0, c0:c1, h], gk[0, c0:c1, h].astype(np.float64),
                            inp["beta"][0, c0:c1, h])
            assert O.parity_err(Akk[0, c0:c1, h, :n], wy["A"], out_bf16=True) <= TOL
            assert O.parity_err(w[0, c0:c1, h], wy["W"], out_bf16=True) <= TOL
            assert O.parity_err(u[0, c0:c1, h], wy["U"], out_bf16=True) <= TOL
            assert O.parity_err(kg[0, c0:c1, h], wy["kg"], out_bf16=True) <= TOL
            qh = inp["q"][0, c0:c1, h].astype(np.float64)
            assert O.parity_err(qg[0, c0:c1, h], qh * wy["gam"], out_bf16=True) <= TOL
            kh = inp["k"][0, c0:c1, h].astype(np.float64)
            gh = gk[0, c0:c1, h].astype(np.float64)
            ref_aqk = np.zeros((n, n))
            for i in range(n):
                for j in range(i + 1):
                    ref_aqk[i, j] = scale * np.sum(qh[i] * kh[j] * np.exp2(gh[i] - gh[j]))
            assert O.parity_err(Aqk[0, c0:c1, h, :n], ref_aqk, out_bf16=True) <= TOL


def test_fwd_h_from_reference_layout(dev):
    """memt_gdn2_fwd_h on bf16 WY tensors vs the oracle scan of the same
    tensors: snapshots at block starts, uncommitted events, final states."""
    T, H, D = 260, 2, 64
    inp = O.synth_inputs(T, H, D, D, seed=51, h0_std=0.05, n_seq=2)
    samples = [0, 120, 260]
    events = [0, 64, 120, 200, 260]
    commit = [1, 0, 1, 1]
    gk = O.chunk_local_cumsum(inp["g"], 64, scale=O.RCP_LN2, cu_seqlens=events)
    oplan = O.build_chunk_plan(samples, samples, event_slice=events, commit_mask=commit)
    w, u, kg = (np.zeros_like(inp[n]) for n in ("k", "v", "k"))
    for h in range(H):
        for c in range(oplan.num_chunk):
            c0 = int(oplan.chunk_tok0[c])
            c1 = c0 + int(oplan.chunk_len[c])
            wy = O.wy_chunk(inp["k"][0, c0:c1, h], inp["v"][0, c0:c1, h], gk[0, c0:c1, h], inp["beta"][0, c0:c1, h])
            w[0, c0:c1, h], u[0, c0:c1, h], kg[0, c0:c1, h] = wy["W"], wy["U"], wy["kg"]
    w, u, kg = (O.bf16_round(x) for x in (w, u, kg))
    gk32 = gk.astype(np.float32)
    plan = memt_gdn2.build_chunk_plan(samples, samples, event_slice=events, commit_mask=commit, device=dev)
    snaps, final = memt_gdn2.memt_gdn2_fwd_h(bf(kg, dev), bf(w, dev), bf(u, dev), to_dev(gk32, dev), plan,
                                             initial_state=to_dev(inp["h0"], dev))
    s_ref, f_ref = O.state_scan(kg, w, u, gk32, oplan, h0=inp["h0"])
    assert O.max_rel_err(host(final), f_ref) <= TOL
    assert np.array_equal(host(snaps), s_ref.astype(np.float32))


def test_read_fwd(dev):
    T, H, D = 150, 2, 128
    lengths = [50, 100]
    rng = np.random.default_rng(61)
    q = O.bf16_round(O.l2norm(rng.standard_normal((1, T, H, D)).astype(np.float32))[0])
    S = (rng.standard_normal((2, H, D, D)) * 0.1).astype(np.float32)
    out = memt_gdn2.snapshot_read(bf(q, dev), to_dev(S, dev), lengths, D ** -0.5, bf16_accumulator_output=True)
    ref = O.snapshot_read(q, S, lengths, D ** -0.5)
    assert O.parity_err(host(out), ref, out_bf16=True) <= TOL


def test_full_size_workload_heads(dev):
    """B=1, H=16, T=8192, d=128, chunk 64: the final state and the causal output
    of every head vs the fp64 chunked oracle (torch port, pinned to the token
    recurrence), inputs drawn as the benchmark draws them."""
    from oracle.gdn2_torch import chunked_gdn2_torch

    T, H, D = 8192, 16, 128
    print("full-size workload B=1 H=16 T=8192 D=128 (all heads)", flush=True)
    t = workload_inputs(T, H, D, seed=20261202)
    o, ht = memt_gdn2.chunk_gdn2(*(t[n].to(dev) for n in ("q", "k", "v", "g", "beta")),
                                 initial_state=t["h0"].to(dev), out_mode="causal")
    o, ht = host(o), host(ht)
    assert np.all(np.isfinite(o)) and np.all(np.isfinite(ht))
    f64 = lambda n: t[n][0].double()  # noqa: E731
    o_ref, h_ref = chunked_gdn2_torch(f64("q"), f64("k"), f64("v"), f64("g"), f64("beta"), h0=t["h0"][0].double(),
                                      out_mode="causal", dtype=torch.float64)
    check("final state (16 heads)", ht[0], h_ref.numpy(), out_bf16=False)
    check("causal output (16 heads)", o[0], o_ref.numpy(), out_bf16=True)
    for h in range(H):
        assert O.max_rel_err(ht[0, h], h_ref[h].numpy()) <= TOL, h


def test_h4_t512_d64_vs_recurrence(dev):
    """The naive-recurrence configuration's exact shape (B=1, H=4, T=512, d=64,
    zero initial state), seeded as the benchmark seeds it, in causal and
    snapshot modes, against the fp64 token recurrence."""
    T, H, D = 512, 4, 64
    print("naive-recurrence shape B=1 H=4 T=512 D=64", flush=True)
    t = workload_inputs(T, H, D, seed=20261201, h0_std=0.0)
    args = [t[n].to(dev) for n in ("q", "k", "v", "g", "beta")]
    ins = {n: t[n].float().numpy() for n in ("q", "k", "v", "g", "beta")}
    for mode in ("causal", "snapshot"):
        o, ht = memt_gdn2.chunk_gdn2(*args, initial_state=t["h0"].to(dev), out_mode=mode)
        o_ref, h_ref = O.recurrent_gdn2(ins["q"], ins["k"], ins["v"], ins["g"], ins["beta"],
                                        h0=t["h0"].numpy(), out_mode=mode)
        check(f"final state ({mode})", host(ht), h_ref, out_bf16=False)
        if mode == "causal":
            check("causal output", host(o), o_ref, out_bf16=True)
        else:  # every token reads the zero initial state
            assert np.all(host(o) == 0.0) and np.all(o_ref == 0.0)


def _segment_lengths(total, n, seed):
    """n lengths drawn uniformly from [1024, 32768], rescaled to sum to total
    (rounded, the last one absorbing the remainder)."""
    rng = np.random.default_rng(seed)
    raw = rng.uniform(1024, 32768, n)
    lengths = [int(round(x)) for x in raw * total / raw.sum()]
    lengths[-1] = total - sum(lengths[:-1])
    return lengths


def test_varlen_full_size_workload(dev):
    """4 packed segments summing to 65536 tokens, H=16, d=128, per-segment
    initial states: every head of every segment against the fp64 chunked torch
    oracle, and every head's final state against each segment run alone."""
    from oracle.gdn2_torch import chunked_gdn2_torch

    T, H, D = 65536, 16, 128
    lengths = _segment_lengths(T, 4, seed=20261204)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    print(f"varlen full size lengths={lengths}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(20261204)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(1, T, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    k = nrm(torch.randn(1, T, H, D, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    v = torch.randn(1, T, H, D, generator=gen, device=dev).to(torch.bfloat16)
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, H, D, generator=gen, device=dev))
    beta = torch.sigmoid(torch.randn(1, T, H, D, generator=gen, device=dev))
    h0 = torch.randn(4, H, D, D, generator=gen, device=dev) * 0.02
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, cu_seqlens=cu, out_mode="causal")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o.float()).all()) and bool(torch.isfinite(ht).all())
    for n in range(4):  # every head of every segment
        a, b = cu[n], cu[n + 1]
        sl = lambda t: t[0, a:b].double().cpu()  # noqa: E731
        o_ref, h_ref = chunked_gdn2_torch(sl(q), sl(k), sl(v), sl(g), sl(beta), h0=h0[n].double().cpu(),
                                          out_mode="causal", dtype=torch.float64)
        check(f"segment {n} ({b - a} tokens) final state", host(ht[n]), h_ref.numpy(), out_bf16=False)
        check(f"segment {n} causal output", host(o[0, a:b]), o_ref.numpy(), out_bf16=True)
        # the segment alone (a different scan grouping): same states within tolerance
        o1, h1 = memt_gdn2.chunk_gdn2(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b],
                                      initial_state=h0[n:n + 1], out_mode="causal")
        assert O.max_rel_err(host(ht[n]), host(h1[0])) <= TOL, n


def test_empty_segments_and_empty_input(dev):
    """A zero-length sequence keeps its initial state; a zero-token launch
    returns an empty output and the initial states unchanged."""
    T, H, D = 250, 2, 64
    cu = [0, 100, 100, 250]
    inp = O.synth_inputs(T, H, D, D, seed=71, h0_std=0.1, n_seq=3)
    q, k, v, g, beta, h0 = _dev_inputs(inp, dev)
    o, ht = memt_gdn2.chunk_gdn2(q, k, v, g, beta, initial_state=h0, cu_seqlens=cu, out_mode="causal")
    o_ref, h_ref = O.recurrent_gdn2(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], h0=inp["h0"],
                                    cu_seqlens=cu)
    assert np.array_equal(host(ht[1]), inp["h0"][1])
    assert O.max_rel_err(host(ht), h_ref) <= TOL
    assert O.parity_err(host(o), o_ref, out_bf16=True) <= TOL
    z = lambda t: t[:, :0].contiguous()  # noqa: E731
    o0, ht0 = memt_gdn2.chunk_gdn2(z(q), z(k), z(v), z(g), z(beta), initial_state=h0[:1], out_mode="causal")
    assert o0.shape == (1, 0, H, D) and torch.equal(ht0, h0[:1])
