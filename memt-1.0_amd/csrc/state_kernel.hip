// Inter-chunk state scan of the chunked GDN-2 update.
//
// One workgroup (4 waves) per (sequence, head, slice of BV state columns).
// Columns of the state are independent in the recurrence (v_new[:, j] only
// depends on S[:, j]), so each workgroup keeps its K x BV fp32 slice of S in
// MFMA accumulators for the whole sequence and walks the chunks in order
// (models/qwen/ops/_triton/state.py:76-115):
//
//   snapshot S if the chunk starts a read block
//   V_new = U - W . bf16(S)                        (bf16 MFMA, erase path)
//   o     = scale * qg . bf16(S) + Aqk . V_new      (causal output, optional)
//   S     = decay * S + kg^T . f16(V_new)           (f16 MFMA, value path, if committed)
//
// Wave w owns S rows [w*K/4, (w+1)*K/4) and V_new / o token rows [16w, 16w+16),
// so it reads only its quarter of each chunk record.  bf16(S) and f16(V_new)
// cross waves through two column-major LDS tiles, with two LDS-only barriers
// per chunk.  The W / qg / kg^T / Aqk records are P-frags, whose reduction
// index pairs with B operands gathered as two 8-byte LDS reads per lane.
//
// Prefetch: everything a chunk needs from global memory (its operand
// fragments and its plan entries) is loaded into registers two chunks ahead;
// the loop is unrolled by two so the two register buffers alternate without
// copies, and the compiler's vmcnt waits stay exact.
#include "gdn2_internal.h"

namespace memt {
namespace {

template <int K, int V, int BV, bool CAUSAL>
struct ScanFrag {
  static constexpr int KS = K / 32;
  static constexpr int RT = K / 64;   // 16-row S tiles per wave
  static constexpr int CT = BV / 16;  // 16-column tiles per workgroup
  bf16x8 w[KS];
  bf16x8 qg[CAUSAL ? KS : 1];
  f16x8 kg[RT][2];
  f16x8 aq[CAUSAL ? 2 : 1];
  f16x4 u[CT];
  f32x4 d[RT];
  int flags, block, tok0, len;
};

template <int K, int V, int BV, bool CAUSAL>
__global__ __launch_bounds__(256) void state_kernel(StateArgs a) {
  using F = ScanFrag<K, V, BV, CAUSAL>;
  constexpr int C = kChunk;
  constexpr int NV = V / BV;
  constexpr int KS = F::KS;
  constexpr int RT = F::RT;
  constexpr int CT = F::CT;
  constexpr int SKP = K + 8;  // pitch of column-major bf16(S)
  constexpr int VNP = C + 8;  // pitch of column-major f16(V_new)
  static_assert(RT >= 1 && CT >= 1, "tile shape");

  __shared__ __attribute__((aligned(16))) __bf16 S_lds[BV * SKP];
  __shared__ __attribute__((aligned(16))) _Float16 Vn_lds[BV * VNP];

  // XCD-aware order: the NV slices of one (sequence, head) share an XCD (and its L2),
  // since they all read the same per-chunk records.
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

  // S tile rt of this wave: rows 16*(w*RT + rt) + 4*lg + e, column v0 + 16*ct + lr
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
  // settle the initial-state loads here: otherwise every later use of S in the
  // loop would wait for all outstanding loads, prefetches included
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  asm volatile("" ::: "memory");

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

  // Plan entries of chunks [mbase, mbase + 64), one chunk per lane, read out
  // with readlane.  Loading them per chunk would make the compiler move each
  // entry to a scalar register right after its load, waiting for every
  // outstanding prefetch; this way the wait comes once per 64 chunks.
  const int c_begin = a.seq_chunk_offsets[n], c_end = a.seq_chunk_offsets[n + 1];
  int mbase = c_begin - 64;
  int m_flags = 0, m_block = -1, m_tok0 = 0, m_len = 0;
  auto meta = [&](int c, F& f) {
    if (c - mbase >= 64) {
      mbase = c;
      const int cc = c + lane;
      const bool ok = cc < c_end;
      m_flags = !ok ? 0 : a.chunk_flags ? a.chunk_flags[cc] : MEMT_GDN2_CHUNK_COMMIT;
      m_block = (ok && a.snaps != nullptr && a.chunk_block_ids != nullptr) ? a.chunk_block_ids[cc] : -1;
      if constexpr (CAUSAL) {
        m_tok0 = ok ? a.chunk_tok0[cc] : 0;
        m_len = ok ? a.chunk_len[cc] : 0;
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    const int i = c - mbase;
    f.flags = __builtin_amdgcn_readlane(m_flags, i);
    f.block = __builtin_amdgcn_readlane(m_block, i);
    f.tok0 = CAUSAL ? __builtin_amdgcn_readlane(m_tok0, i) : 0;
    f.len = CAUSAL ? __builtin_amdgcn_readlane(m_len, i) : 0;
  };

  auto load = [&](int c, F& f) {
    meta(c, f);
    const size_t unit = (size_t)c * H + h;
    const __bf16* Wp = a.in.W + unit * (size_t)(C * K);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const size_t fo = ((size_t)(w * KS + s) * 64 + lane) * 8;
      f.w[s] = *(const bf16x8*)(Wp + fo);
      if constexpr (CAUSAL) f.qg[s] = *(const bf16x8*)(a.in.qg + unit * (size_t)(C * K) + fo);
    }
    const _Float16* Kp = a.in.kgT + unit * (size_t)(C * K);
    const float* dp = a.in.decay + unit * K;
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
    }
    const _Float16* Up = a.in.U + unit * (size_t)(C * V);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
      f.u[ct] = *(const f16x4*)(Up + ((size_t)(w * (V / 16) + (v0 >> 4) + ct) * 64 + lane) * 4);
  };

  // B operand of a P-frag product: rows {32s + 4lg + e} and {32s + 16 + 4lg + e}
  // of a column-major tile (column 16*ct + lr), as two 8-byte reads.
  auto b_operand = [&](const auto* tile, int pitch, int ct, int s) {
    using T = std::remove_cv_t<std::remove_pointer_t<decltype(tile)>>;
    typedef T T4 __attribute__((ext_vector_type(4)));
    typedef T T8 __attribute__((ext_vector_type(8)));
    const T* col = tile + (16 * ct + lr) * pitch + 32 * s + 4 * lg;
    const T4 lo = *(const T4*)col;
    const T4 hi = *(const T4*)(col + 16);
    return T8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  auto step = [&](const F& f) {
    if (f.block >= 0 && (f.flags & MEMT_GDN2_CHUNK_BLOCK_START)) {
      const size_t soff = ((size_t)f.block * H + h) * K * V;
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
    // ---- V_new (and qg . S) for token rows [16w, 16w + 16) ----
    f32x4 acc[CT], acco[CAUSAL ? CT : 1];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      acc[ct] = zero4();
      if constexpr (CAUSAL) acco[ct] = zero4();
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const bf16x8 sb = b_operand(S_lds, SKP, ct, s);
        acc[ct] = mfma_bf16(f.w[s], sb, acc[ct]);
        if constexpr (CAUSAL) acco[ct] = mfma_bf16(f.qg[s], sb, acco[ct]);
      }
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      f16x4 vn;
#pragma unroll
      for (int e = 0; e < 4; ++e) vn[e] = (_Float16)((float)f.u[ct][e] - acc[ct][e]);
      *(f16x4*)(&Vn_lds[(16 * ct + lr) * VNP + 16 * w + 4 * lg]) = vn;
    }
    lds_barrier();

    // ---- S = decay * S + kg^T . V_new; causal output ----
    f16x8 vb[CT][2];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int s = 0; s < 2; ++s) vb[ct][s] = b_operand(Vn_lds, VNP, ct, s);
    if (f.flags & MEMT_GDN2_CHUNK_COMMIT) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
          for (int e = 0; e < 4; ++e) S[rt][ct][e] *= f.d[rt][e];
#pragma unroll
          for (int s = 0; s < 2; ++s) S[rt][ct] = mfma_f16(f.kg[rt][s], vb[ct][s], S[rt][ct]);
        }
      }
    }
    if constexpr (CAUSAL) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acco[ct][e] *= a.scale;
#pragma unroll
        for (int s = 0; s < 2; ++s) acco[ct] = mfma_f16(f.aq[s], vb[ct][s], acco[ct]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = 16 * w + 4 * lg + e;
          if (t < f.len) a.o[((size_t)(f.tok0 + t) * H + h) * V + v0 + 16 * ct + lr] = (__bf16)acco[ct][e];
        }
      }
    }
    write_S_lds();
    lds_barrier();
  };

  write_S_lds();
  lds_barrier();

  // The prefetches past the last chunk reload the last chunk (in bounds and
  // unused): unconditional loads keep the compiler's vmcnt waits exact.
  if (c_begin < c_end) {
    const int c_last = c_end - 1;
    F fa, fb;
    load(c_begin, fa);
    load(min(c_begin + 1, c_last), fb);
    for (int c = c_begin; c < c_end; c += 2) {
      step(fa);
      load(min(c + 2, c_last), fa);
      if (c + 1 >= c_end) break;
      step(fb);
      load(min(c + 3, c_last), fb);
    }
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
