"""Write the seeded golden fixtures of the GDN-2 memory path.

The reference ships no golden vectors for this path, so these fixtures are
produced by the oracle (oracle/gdn2.py, fp64 token recurrence) from seeded
inputs.  They are regression vectors: the CPU tests recompute them, and the
GPU tests compare the HIP kernels against them.

Run: python tests/golden/make_golden.py   (writes tests/golden/*.npz)
"""

from pathlib import Path
import sys

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import gdn2 as O  # noqa: E402

OUT = Path(__file__).resolve().parent


def bf16_bits(x):
    return (O.bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def update_fixture():
    # two packed sequences, 64-dim heads, write events every 48 tokens
    T, H, D = 160, 2, 64
    cu = [0, 70, 160]
    inp = O.synth_inputs(T, H, D, D, seed=20261201, h0_std=0.05, n_seq=2)
    args = [inp[n] for n in ("q", "k", "v", "g", "beta")]
    o_c, h_c = O.recurrent_gdn2(*args, h0=inp["h0"], cu_seqlens=cu, out_mode="causal")
    np.savez_compressed(
        OUT / "gdn2_update_small.npz",
        cu_seqlens=np.array(cu, np.int32), chunk_tokens=np.int32(48),
        q=bf16_bits(inp["q"]), k=bf16_bits(inp["k"]), v=bf16_bits(inp["v"]),
        g=inp["g"], beta=inp["beta"], h0=inp["h0"],
        o_causal=o_c.astype(np.float32), ht=h_c.astype(np.float32),
    )


def readout_fixture():
    B, H, D = 4, 2, 64
    rng = np.random.default_rng(20261202)
    S = (rng.standard_normal((B, H, D, D)) * 0.02).astype(np.float32)
    q = O.bf16_round(O.l2norm(rng.standard_normal((B, H, D)).astype(np.float32))[0])
    gate = O.bf16_round(rng.standard_normal((B, H, D)).astype(np.float32))
    w = O.bf16_round((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    out = O.readout_fused(S, q, gate, w, scale=D ** -0.5, eps=1e-6)
    out_sig = O.readout_fused(S, q, gate, w, scale=D ** -0.5, eps=1e-6, gate_kind="sigmoid")
    np.savez_compressed(OUT / "gdn2_readout_small.npz", S=S, q=bf16_bits(q), gate=bf16_bits(gate), w=bf16_bits(w),
                        out_softcap=out.astype(np.float32), out_sigmoid=out_sig.astype(np.float32))


def plan_fixture():
    lengths = [130, 1, 129, 3000]
    p = O.packed_plan(lengths, chunk_tokens=2048)
    np.savez_compressed(OUT / "plan_packed.npz", lengths=np.array(lengths, np.int64), chunk_tokens=np.int64(2048),
                        **{k: getattr(p, k) for k in ("event_slice", "chunk_indices", "sample_chunk_offsets",
                                                      "chunk_block_ids", "chunk_is_block_start", "chunk_tok0",
                                                      "chunk_len", "chunk_commits")})


if __name__ == "__main__":
    update_fixture()
    readout_fixture()
    plan_fixture()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
