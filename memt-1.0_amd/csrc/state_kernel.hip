// Inter-chunk state scan of the chunked GDN-2 update.
//
// One workgroup per (sequence, head, V slice of BV columns).  Columns of the
// state are independent in the recurrence (v_new[:, j] only depends on
// S[:, j]), so each workgroup keeps its K x BV fp32 slice of S in MFMA
// accumulators for the whole sequence and walks the chunks in order
// (models/qwen/ops/_triton/state.py:76-115):
//
//   snapshot S if the chunk starts a read block
//   V_new = U - W . bf16(S)                        (bf16 MFMA, erase path)
//   o     = scale * qg . bf16(S) + Aqk . V_new      (causal output, optional)
//   S     = decay * S + kg^T . f16(V_new)           (f16 MFMA, value path, if committed)
//
// Wave w owns S rows [w*K/4, (w+1)*K/4) and V_new / o token rows [16w, 16w+16).
// Two LDS buffers carry bf16(S) (column-major) and f16(V_new) (column-major)
// between waves; two barriers per chunk.
#include "gdn2_internal.h"

namespace memt {
namespace {

template <int K, int V, int BV, bool CAUSAL>
__global__ __launch_bounds__(256) void state_kernel(StateArgs a) {
  constexpr int C = kChunk;
  constexpr int NV = V / BV;
  constexpr int CT = BV / 16;        // column tiles per workgroup
  constexpr int RT = K / 64;         // 16-row tiles of S per wave
  constexpr int SKP = K + 8;         // pitch of column-major bf16(S)
  constexpr int VNP = C + 8;         // pitch of column-major f16(V_new)
  static_assert(RT >= 1 && CT >= 1, "tile shape");

  __shared__ __attribute__((aligned(16))) __bf16 S_lds[BV * SKP];
  __shared__ __attribute__((aligned(16))) _Float16 Vn_lds[BV * VNP];

  // XCD-aware order: the NV slices of one (sequence, head) share an XCD (and its L2),
  // since they all read the same per-chunk W / kg / qg / Aqk records.
  const int total = gridDim.x;
  int bid = blockIdx.x;
  if ((total & 7) == 0) bid = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int vs = bid % NV;
  const int h = (bid / NV) % a.H;
  const int n = bid / (NV * a.H);
  const int H = a.H;
  const int v0 = vs * BV;

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  // S rows of tile rt of this wave: 16*(w*RT + rt) + 4*lg + e, column v0 + 16*ct + lr
  f32x4 S[RT][CT];
  const size_t state_off = ((size_t)n * H + h) * K * V;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (w * RT + rt) + 4 * lg + e;
        S[rt][ct][e] = a.h0 ? a.h0[state_off + (size_t)row * V + v0 + 16 * ct + lr] : 0.f;
      }

  auto write_S_lds = [&]() {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        bf16x4 b4;
#pragma unroll
        for (int e = 0; e < 4; ++e) b4[e] = (__bf16)S[rt][ct][e];
        *(bf16x4*)(&S_lds[(16 * ct + lr) * SKP + 16 * (w * RT + rt) + 4 * lg]) = b4;
      }
  };
  write_S_lds();
  __syncthreads();

  // Everything a chunk needs from global memory, loaded one chunk ahead so the
  // loads of chunk c+1 are in flight while chunk c computes.
  struct Frag {
    bf16x8 w[K / 32];
    bf16x8 qg[CAUSAL ? K / 32 : 1];
    f16x4 u[CT];
    f32x4 d[RT];
    f16x8 kg[RT][2];
    f16x8 aq[CAUSAL ? 2 : 1];
    int flags, block, tok0, len;
  };
  auto load_frag = [&](int c, Frag& f) {
    const size_t unit = (size_t)c * H + h;
    const __bf16* Wp = a.in.W + unit * (size_t)(C * K);
#pragma unroll
    for (int s = 0; s < K / 32; ++s) {
      const size_t fo = ((size_t)(w * (K / 32) + s) * 64 + lane) * 8;
      f.w[s] = *(const bf16x8*)(Wp + fo);
      if constexpr (CAUSAL) f.qg[s] = *(const bf16x8*)(a.in.qg + unit * (size_t)(C * K) + fo);
    }
    const _Float16* Up = a.in.U + unit * (size_t)(C * V);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
      f.u[ct] = *(const f16x4*)(Up + ((size_t)(w * (V / 16) + (v0 >> 4) + ct) * 64 + lane) * 4);
    const float* dp = a.in.decay + unit * K;
    const _Float16* Kp = a.in.kgT + unit * (size_t)(C * K);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rtile = w * RT + rt;
      f.d[rt] = *(const f32x4*)(dp + 16 * rtile + 4 * lg);
#pragma unroll
      for (int s = 0; s < 2; ++s) f.kg[rt][s] = *(const f16x8*)(Kp + ((size_t)(rtile * 2 + s) * 64 + lane) * 8);
    }
    if constexpr (CAUSAL) {
      const _Float16* Ap = a.in.Aqk + unit * (size_t)(C * C);
#pragma unroll
      for (int s = 0; s < 2; ++s) f.aq[s] = *(const f16x8*)(Ap + ((size_t)(w * 2 + s) * 64 + lane) * 8);
      f.tok0 = a.chunk_tok0[c];
      f.len = a.chunk_len[c];
    }
    f.flags = a.chunk_flags ? a.chunk_flags[c] : MEMT_GDN2_CHUNK_COMMIT;
    f.block = (a.snaps != nullptr && (f.flags & MEMT_GDN2_CHUNK_BLOCK_START)) ? a.chunk_block_ids[c] : -1;
  };

  const int c_begin = a.seq_chunk_offsets[n], c_end = a.seq_chunk_offsets[n + 1];
  Frag cur, nxt;
  if (c_begin < c_end) load_frag(c_begin, cur);
  for (int c = c_begin; c < c_end; ++c) {
    if (c + 1 < c_end) load_frag(c + 1, nxt);
    if (cur.block >= 0) {
      const size_t soff = ((size_t)cur.block * H + h) * K * V;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = 16 * (w * RT + rt) + 4 * lg + e;
            a.snaps[soff + (size_t)row * V + v0 + 16 * ct + lr] = S[rt][ct][e];
          }
    }

    // ---- phase 1: V_new (and qg . S) for token rows [16w, 16w + 16) ----
    f32x4 acc[CT], acco[CAUSAL ? CT : 1];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      acc[ct] = zero4();
      if constexpr (CAUSAL) acco[ct] = zero4();
    }
#pragma unroll
    for (int s = 0; s < K / 32; ++s) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const bf16x8 sb = *(const bf16x8*)(&S_lds[(16 * ct + lr) * SKP + 32 * s + 8 * lg]);
        acc[ct] = mfma_bf16(cur.w[s], sb, acc[ct]);
        if constexpr (CAUSAL) acco[ct] = mfma_bf16(cur.qg[s], sb, acco[ct]);
      }
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      f16x4 vn;
#pragma unroll
      for (int e = 0; e < 4; ++e) vn[e] = (_Float16)((float)cur.u[ct][e] - acc[ct][e]);
      *(f16x4*)(&Vn_lds[(16 * ct + lr) * VNP + 16 * w + 4 * lg]) = vn;
    }
    __syncthreads();

    // ---- phase 2: state update and causal output ----
    if (cur.flags & MEMT_GDN2_CHUNK_COMMIT) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e) S[rt][ct][e] *= cur.d[rt][e];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            const f16x8 vb = *(const f16x8*)(&Vn_lds[(16 * ct + lr) * VNP + 32 * s + 8 * lg]);
            S[rt][ct] = mfma_f16(cur.kg[rt][s], vb, S[rt][ct]);
          }
        }
      }
    }
    if constexpr (CAUSAL) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) acco[ct][e] *= a.scale;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const f16x8 vb = *(const f16x8*)(&Vn_lds[(16 * ct + lr) * VNP + 32 * s + 8 * lg]);
          acco[ct] = mfma_f16(cur.aq[s], vb, acco[ct]);
        }
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = 16 * w + 4 * lg + e;
          if (t < cur.len)
            a.o[((size_t)(cur.tok0 + t) * H + h) * V + v0 + 16 * ct + lr] = (__bf16)acco[ct][e];
        }
    }
    write_S_lds();
    __syncthreads();
    cur = nxt;
  }

  if (a.ht != nullptr) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * (w * RT + rt) + 4 * lg + e;
          a.ht[state_off + (size_t)row * V + v0 + 16 * ct + lr] = S[rt][ct][e];
        }
  }
}

template <int K, int V, int BV>
hipError_t launch_t(const StateArgs& a, bool causal, hipStream_t stream) {
  dim3 grid((V / BV) * a.H * a.n_seq), block(256);
  if (causal)
    hipLaunchKernelGGL((state_kernel<K, V, BV, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((state_kernel<K, V, BV, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_state(const StateArgs& a, int K, int V, bool causal, hipStream_t stream) {
  if (a.n_seq == 0) return hipSuccess;
  if (K == 64 && V == 64) return launch_t<64, 64, 32>(a, causal, stream);
  if (K == 128 && V == 128) return launch_t<128, 128, 32>(a, causal, stream);
  return hipErrorInvalidValue;
}

}  // namespace memt
