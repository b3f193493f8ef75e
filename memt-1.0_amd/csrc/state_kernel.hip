// Inter-chunk state scan of the chunked GDN-2 update.
//
// One workgroup (8 waves) per (sequence or chunk group, head) holds the head's
// whole K x NC fp32 state in MFMA accumulators and walks the chunks in order
// (models/qwen/ops/_triton/state.py:76-115):
//
//   snapshot S if the chunk starts a read block
//   V_new = U - W . f16(S)                         (erase path)
//   o     = scale * qg . f16(S) + Aqk . V_new       (causal output, optional)
//   S     = decay * S + kg^T . f16(V_new)           (value path, if committed)
// Every product is fp16 MFMA with fp32 accumulation; S stays fp32.
//
// Wave w = 4 c + q owns state rows [q K/4, (q+1) K/4), token rows [16 q, 16 q + 16)
// and the column half c.  The two waves of a (q, c) pair on one SIMD read the
// same chunk record fragments (W / qg / kg^T / Aqk rows of quarter q), so each
// record is fetched from L2 once per head and chunk and the second read hits
// the CU's L1.  f16(S) and f16(V_new) cross waves through two column-major
// LDS tiles, with two LDS-only barriers per chunk.  The records are P-frags,
// whose reduction index pairs with B operands gathered as two 8-byte LDS reads.
//
// The causal output is formed transposed (f16(S) and V_new as A operands, qg
// and Aqk as B operands), so each lane holds 4 consecutive output columns of
// one token and stores 8 bytes.
//
// Prefetch: each record fragment of chunk c + 1 is loaded right after its last
// use in chunk c (one register buffer); plan entries come from a per-wave
// cache of 64 chunks.  Loads past the last chunk reload the last chunk, so
// every load is unconditional and the compiler's vmcnt waits stay exact.
//
// Long sequences use a two-level scan over groups of chunks (the recurrence is
// linear in S): the same loop first runs on [I | 0] per group to form the
// group transition P_g and its zero-start contribution Q_g (modes 1 and 2,
// trans_kernel), combine_kernel then chains S_{g+1} = P_g S_g + Q_g per
// sequence (split-bf16 MFMA, ~2^-16 relative), and the scan proper runs per
// group from S_g.
#include "gdn2_internal.h"

namespace memt {
namespace {

template <int K, int NC, bool CAUSAL>
struct ScanFrag {
  static constexpr int KS = K / 32;
  static constexpr int RT = K / 64;    // 16-row state tiles per wave
  static constexpr int CT = NC / 32;   // 16-column tiles per wave (half the columns)
  f16x8 w[KS];
  f16x8 qg[CAUSAL ? KS : 1];
  f16x8 kg[RT][2];
  f16x8 aq[CAUSAL ? 2 : 1];
  f16x4 u[CT];
  f32x4 d[RT];
};

constexpr int kScanThreads = 512;

// MODE 0: the scan (per sequence, or per group from its start state), NC = V
// MODE 1: group transition P_g, columns of the K x K identity, no values, NC = K
// MODE 2: group contribution Q_g, value columns from a zero state, NC = V
template <int K, int V, int NC, bool CAUSAL, int MODE>
__device__ __forceinline__ void scan_body(const StateArgs& a, int unitg, int h, _Float16* S_lds,
                                          _Float16* Vn_lds) {
  using F = ScanFrag<K, NC, CAUSAL>;
  constexpr int C = kChunk;
  constexpr int KS = F::KS, RT = F::RT, CT = F::CT;
  constexpr int SKP = K + 8;  // pitch of column-major f16(S)
  constexpr int VNP = C + 8;  // pitch of column-major f16(V_new)
  static_assert(MODE == 0 || !CAUSAL, "the transition modes write no output");
  static_assert(RT >= 1 && CT >= 1, "tile shape");
  const int H = a.H;

  int c_begin, c_end, seq = unitg;
  bool first = true, last = true;
  if (a.group_L == 0) {
    c_begin = a.seq_chunk_offsets[seq];
    c_end = a.seq_chunk_offsets[seq + 1];
  } else {
    if (unitg >= a.grp.seq_group_offsets[a.n_seq]) return;
    seq = a.grp.group_seq[unitg];
    c_begin = a.grp.group_chunk_offsets[unitg];
    c_end = a.grp.group_chunk_offsets[unitg + 1];
    first = unitg == a.grp.seq_group_offsets[seq];
    last = unitg + 1 == a.grp.seq_group_offsets[seq + 1];
    if (MODE != 0 && last) return;  // the last group's transition is never used
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = w & 3, half = w >> 2;
  const int lr = lane & 15, lg = lane >> 4;
  const int col0 = half * (NC / 2);  // first state column of this wave

  // S tile (rt, ct): rows 16 (q RT + rt) + 4 lg + e, column col0 + 16 ct + lr
  f32x4 S[RT][CT];
  const float* h0p = nullptr;
  if constexpr (MODE == 0) {
    if (!first) h0p = a.grp.S0 + ((size_t)unitg * H + h) * K * V;
    else if (a.h0 != nullptr) h0p = a.h0 + ((size_t)seq * H + h) * K * V;
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (q * RT + rt) + 4 * lg + e;
        const int col = col0 + 16 * ct + lr;
        if constexpr (MODE == 1) S[rt][ct][e] = row == col ? 1.f : 0.f;
        else S[rt][ct][e] = h0p ? h0p[(size_t)row * V + col] : 0.f;
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
        f16x4 b4;
#pragma unroll
        for (int e = 0; e < 4; ++e) b4[e] = (_Float16)S[rt][ct][e];
        *(f16x4*)(&S_lds[(col0 + 16 * ct + lr) * SKP + 16 * (q * RT + rt) + 4 * lg]) = b4;
      }
  };

  // Plan entries of chunks [mbase, mbase + 64), one chunk per lane, read out
  // with readlane.  Loading them per chunk would make the compiler move each
  // entry to a scalar register right after its load, waiting for every
  // outstanding prefetch; this way the wait comes once per 64 chunks.
  int mbase = c_begin - 64;
  int m_flags = 0, m_block = -1, m_tok0 = 0, m_len = 0;
  int flags = 0, block = -1, tok0 = 0, len = 0;
  auto meta = [&](int c) {
    if (c - mbase >= 64) {
      mbase = c;
      const int cc = c + lane;
      const bool ok = cc < c_end;
      m_flags = !ok ? 0 : a.chunk_flags ? a.chunk_flags[cc] : MEMT_GDN2_CHUNK_COMMIT;
      m_block = (MODE == 0 && ok && a.snaps != nullptr && a.chunk_block_ids != nullptr) ? a.chunk_block_ids[cc] : -1;
      if constexpr (CAUSAL) {
        m_tok0 = ok ? a.chunk_tok0[cc] : 0;
        m_len = ok ? a.chunk_len[cc] : 0;
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    const int i = c - mbase;
    flags = __builtin_amdgcn_readlane(m_flags, i);
    block = __builtin_amdgcn_readlane(m_block, i);
    tok0 = CAUSAL ? __builtin_amdgcn_readlane(m_tok0, i) : 0;
    len = CAUSAL ? __builtin_amdgcn_readlane(m_len, i) : 0;
  };

  F f;
  // fragments used by the V_new / qg . S products
  auto load_a = [&](int c) {
    const size_t unit = (size_t)c * H + h;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const size_t fo = unit * (size_t)(C * K) + ((size_t)(q * KS + s) * 64 + lane) * 8;
      f.w[s] = *(const f16x8*)(a.in.W + fo);
      if constexpr (CAUSAL) f.qg[s] = *(const f16x8*)(a.in.qg + fo);
    }
    if constexpr (MODE != 1) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        f.u[ct] = *(const f16x4*)(a.in.U + unit * (size_t)(C * V) +
                                  ((size_t)(q * (V / 16) + (col0 >> 4) + ct) * 64 + lane) * 4);
    } else {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) f.u[ct] = f16x4{};
    }
  };
  // fragments used by the state update and the causal output
  auto load_b = [&](int c) {
    const size_t unit = (size_t)c * H + h;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rtile = q * RT + rt;
      f.d[rt] = *(const f32x4*)(a.in.decay + unit * K + 16 * rtile + 4 * lg);
#pragma unroll
      for (int s = 0; s < 2; ++s)
        f.kg[rt][s] = *(const f16x8*)(a.in.kgT + unit * (size_t)(C * K) + ((size_t)(rtile * 2 + s) * 64 + lane) * 8);
    }
    if constexpr (CAUSAL) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
        f.aq[s] = *(const f16x8*)(a.in.Aqk + unit * (size_t)(C * C) + ((size_t)(q * 2 + s) * 64 + lane) * 8);
    }
  };

  // B operand of a P-frag product: rows {32s + 4lg + e} and {32s + 16 + 4lg + e}
  // of a column-major tile (column col, 16 * ct + lr), as two 8-byte reads.
  auto b_operand = [&](const _Float16* tile, int pitch, int col, int s) {
    const _Float16* p = tile + col * pitch + 32 * s + 4 * lg;
    const f16x4 lo = *(const f16x4*)p;
    const f16x4 hi = *(const f16x4*)(p + 16);
    return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  write_S_lds();
  lds_barrier();
  if (c_begin < c_end) {
    const int c_last = c_end - 1;
    meta(c_begin);
    load_a(c_begin);
    load_b(c_begin);
    for (int c = c_begin; c < c_end; ++c) {
      const int cn = min(c + 1, c_last);
      if constexpr (MODE == 0) {
        if (block >= 0 && (flags & MEMT_GDN2_CHUNK_BLOCK_START)) {
          const size_t soff = ((size_t)block * H + h) * K * V;
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int row = 16 * (q * RT + rt) + 4 * lg + e;
                a.snaps[soff + (size_t)row * V + col0 + 16 * ct + lr] = S[rt][ct][e];
              }
        }
      }
      // ---- V_new (token rows 16 q .. 16 q + 15) and o^T from f16(S) ----
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
          const f16x8 sb = b_operand(S_lds, SKP, col0 + 16 * ct + lr, s);
          acc[ct] = mfma_f16(f.w[s], sb, acc[ct]);
          if constexpr (CAUSAL) acco[ct] = mfma_f16(sb, f.qg[s], acco[ct]);
        }
      }
      f16x4 un[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) un[ct] = f.u[ct];
      const int cur_flags = flags, cur_tok0 = tok0, cur_len = len;
      meta(cn);
      load_a(cn);  // W, qg and U of the next chunk
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        f16x4 vn;
#pragma unroll
        for (int e = 0; e < 4; ++e) vn[e] = (_Float16)((float)un[ct][e] - acc[ct][e]);
        *(f16x4*)(&Vn_lds[(col0 + 16 * ct + lr) * VNP + 16 * q + 4 * lg]) = vn;
      }
      lds_barrier();

      // ---- S = decay * S + kg^T . V_new; causal output ----
      f16x8 vb[CT][2];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int s = 0; s < 2; ++s) vb[ct][s] = b_operand(Vn_lds, VNP, col0 + 16 * ct + lr, s);
      if (cur_flags & MEMT_GDN2_CHUNK_COMMIT) {
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
          for (int s = 0; s < 2; ++s) acco[ct] = mfma_f16(vb[ct][s], f.aq[s], acco[ct]);
        }
      }
      load_b(cn);  // decay, kg^T and Aqk of the next chunk
      if constexpr (CAUSAL) {
        // lane holds o[16 q + lr][col0 + 16 ct + 4 lg + e]
        const int t = 16 * q + lr;
        if (t < cur_len) {
          __bf16* orow = a.o + ((size_t)(cur_tok0 + t) * H + h) * V + col0 + 4 * lg;
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            bf16x4 o4;
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = (__bf16)acco[ct][e];
            *(bf16x4*)(orow + 16 * ct) = o4;
          }
        }
      }
      write_S_lds();
      lds_barrier();
    }
  }

  float* out = nullptr;
  if constexpr (MODE == 1) out = a.grp.P + ((size_t)unitg * H + h) * K * K;
  else if constexpr (MODE == 2) out = a.grp.Q + ((size_t)unitg * H + h) * K * V;
  else if (last && a.ht != nullptr) out = a.ht + ((size_t)seq * H + h) * K * V;
  if (out != nullptr) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * (q * RT + rt) + 4 * lg + e;
          out[(size_t)row * NC + col0 + 16 * ct + lr] = S[rt][ct][e];
        }
  }
}

template <int K, int V, bool CAUSAL>
__global__ __launch_bounds__(kScanThreads) void state_kernel(StateArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 S_lds[V * (K + 8)];
  __shared__ __attribute__((aligned(16))) _Float16 Vn_lds[V * (kChunk + 8)];
  scan_body<K, V, V, CAUSAL, 0>(a, blockIdx.x / a.H, blockIdx.x % a.H, S_lds, Vn_lds);
}

// Phase 1 of the two-level scan: blocks [0, units H) form P_g, the rest Q_g.
template <int K, int V>
__global__ __launch_bounds__(kScanThreads) void trans_kernel(StateArgs a, int units) {
  constexpr int NCM = K > V ? K : V;
  __shared__ __attribute__((aligned(16))) _Float16 S_lds[NCM * (K + 8)];
  __shared__ __attribute__((aligned(16))) _Float16 Vn_lds[NCM * (kChunk + 8)];
  const int b = blockIdx.x, per = units * a.H;
  if (b < per)
    scan_body<K, V, K, false, 1>(a, b / a.H, b % a.H, S_lds, Vn_lds);
  else
    scan_body<K, V, V, false, 2>(a, (b - per) / a.H, (b - per) % a.H, S_lds, Vn_lds);
}

// Group table of the two-level scan: sequence n's chunks [c0, c1) form
// ceil((c1 - c0) / L) groups of L chunks (the last one shorter).  One workgroup.
__global__ __launch_bounds__(256) void group_table_kernel(const int32_t* __restrict__ seq_chunk_offsets, int n_seq,
                                                          int L, int32_t* __restrict__ seq_group_offsets,
                                                          int32_t* __restrict__ group_chunk_offsets,
                                                          int32_t* __restrict__ group_seq) {
  __shared__ int scan_s[256];
  __shared__ int carry_s;
  const int tid = threadIdx.x;
  if (tid == 0) carry_s = 0;
  __syncthreads();
  for (int base = 0; base < n_seq; base += 256) {
    const int n = base + tid;
    const int c0 = n < n_seq ? seq_chunk_offsets[n] : 0;
    const int c1 = n < n_seq ? seq_chunk_offsets[n + 1] : 0;
    const int cnt = n < n_seq ? (c1 - c0 + L - 1) / L : 0;
    scan_s[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int add = tid >= off ? scan_s[tid - off] : 0;
      __syncthreads();
      scan_s[tid] += add;
      __syncthreads();
    }
    const int first = carry_s + scan_s[tid] - cnt;
    if (n < n_seq) {
      seq_group_offsets[n] = first;
      for (int j = 0; j < cnt; ++j) {
        group_chunk_offsets[first + j] = c0 + j * L;
        group_seq[first + j] = n;
      }
    }
    __syncthreads();
    if (tid == 0) carry_s += scan_s[255];
    __syncthreads();
  }
  if (tid == 0) {
    seq_group_offsets[n_seq] = carry_s;
    group_chunk_offsets[carry_s] = seq_chunk_offsets[n_seq];
  }
}

// Phase 2 of the two-level scan, one workgroup per (sequence, head, 32 state
// columns): S_{g+1} = P_g S_g + Q_g over the sequence's groups, writing the state
// entering every group but the first.  P_g S_g is split-bf16 MFMA
// (P_hi S_hi + P_hi S_lo + P_lo S_hi) with fp32 accumulation; P and Q of the
// next group are prefetched while the current one is applied.
template <int K, int V>
struct CombineFrag {
  static constexpr int RT = K / 64, KS = K / 32;
  f32x4 p[RT][KS][2];
  f32x4 q[RT][2];
};

template <int K, int V>
__global__ __launch_bounds__(256) void combine_kernel(StateArgs a) {
  using F = CombineFrag<K, V>;
  constexpr int BV = 32, NV = V / BV, RT = F::RT, KS = F::KS, CT = 2, SP = K + 8;
  __shared__ __attribute__((aligned(16))) __bf16 Shi[BV * SP];
  __shared__ __attribute__((aligned(16))) __bf16 Slo[BV * SP];
  const int H = a.H;
  const int vs = blockIdx.x % NV, h = (blockIdx.x / NV) % H, n = blockIdx.x / (NV * H);
  const int g0 = a.grp.seq_group_offsets[n], g1 = a.grp.seq_group_offsets[n + 1];
  if (g1 - g0 <= 1) return;
  const int v0 = vs * BV, tid = threadIdx.x, w = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;

  f32x4 S[RT][CT];
  const float* h0p = a.h0 ? a.h0 + ((size_t)n * H + h) * K * V : nullptr;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * (w * RT + rt) + 4 * lg + e;
        S[rt][ct][e] = h0p ? h0p[(size_t)row * V + v0 + 16 * ct + lr] : 0.f;
      }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): settle h0 before the prefetching loop
  asm volatile("" ::: "memory");

  auto load = [&](int g, F& f) {
    const float* P = a.grp.P + ((size_t)g * H + h) * K * K;
    const float* Q = a.grp.Q + ((size_t)g * H + h) * K * V;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = 16 * (w * RT + rt) + lr;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        f.p[rt][s][0] = *(const f32x4*)(P + (size_t)row * K + 32 * s + 8 * lg);
        f.p[rt][s][1] = *(const f32x4*)(P + (size_t)row * K + 32 * s + 8 * lg + 4);
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          f.q[rt][ct][e] = Q[(size_t)(16 * (w * RT + rt) + 4 * lg + e) * V + v0 + 16 * ct + lr];
    }
  };
  auto step = [&](int g, const F& f) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        bf16x4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hi[e] = (__bf16)S[rt][ct][e];
          lo[e] = (__bf16)(S[rt][ct][e] - (float)hi[e]);
        }
        const int off = (16 * ct + lr) * SP + 16 * (w * RT + rt) + 4 * lg;
        *(bf16x4*)(&Shi[off]) = hi;
        *(bf16x4*)(&Slo[off]) = lo;
      }
    lds_barrier();
    f32x4 acc[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = zero4();
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8 bh[CT], bl[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        bh[ct] = *(const bf16x8*)(&Shi[(16 * ct + lr) * SP + 32 * s + 8 * lg]);
        bl[ct] = *(const bf16x8*)(&Slo[(16 * ct + lr) * SP + 32 * s + 8 * lg]);
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        bf16x8 ph, pl;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float pv = f.p[rt][s][i >> 2][i & 3];
          ph[i] = (__bf16)pv;
          pl[i] = (__bf16)(pv - (float)ph[i]);
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          acc[rt][ct] = mfma_bf16(ph, bh[ct], acc[rt][ct]);
          acc[rt][ct] = mfma_bf16(ph, bl[ct], acc[rt][ct]);
          acc[rt][ct] = mfma_bf16(pl, bh[ct], acc[rt][ct]);
        }
      }
    }
    float* S0 = a.grp.S0 + ((size_t)(g + 1) * H + h) * K * V;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          S[rt][ct][e] = acc[rt][ct][e] + f.q[rt][ct][e];
          S0[(size_t)(16 * (w * RT + rt) + 4 * lg + e) * V + v0 + 16 * ct + lr] = S[rt][ct][e];
        }
    lds_barrier();
  };
  // groups g0 .. g1 - 2 each produce the start state of the next group
  const int glast = g1 - 2;
  F fa, fb;
  load(g0, fa);
  load(min(g0 + 1, glast), fb);
  for (int g = g0; g <= glast; g += 2) {
    step(g, fa);
    load(min(g + 2, glast), fa);
    if (g + 1 > glast) break;
    step(g + 1, fb);
    load(min(g + 3, glast), fb);
  }
}

template <int K, int V>
hipError_t launch_t(const StateArgs& a, bool causal, hipStream_t stream) {
  int units = a.n_seq;
  if (a.group_L > 0) {
    units = group_bound(a.n_chunk, a.n_seq, a.group_L);
    hipLaunchKernelGGL(group_table_kernel, dim3(1), dim3(256), 0, stream, a.seq_chunk_offsets, a.n_seq, a.group_L,
                       a.grp.seq_group_offsets, a.grp.group_chunk_offsets, a.grp.group_seq);
    hipLaunchKernelGGL((trans_kernel<K, V>), dim3(2 * units * a.H), dim3(kScanThreads), 0, stream, a, units);
    hipLaunchKernelGGL((combine_kernel<K, V>), dim3((V / 32) * a.H * a.n_seq), dim3(256), 0, stream, a);
  }
  const dim3 grid(units * a.H), block(kScanThreads);
  if (causal)
    hipLaunchKernelGGL((state_kernel<K, V, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((state_kernel<K, V, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_state(const StateArgs& a, int K, int V, bool causal, hipStream_t stream) {
  if (a.n_seq == 0) return hipSuccess;
  if (K == 64 && V == 64) return launch_t<64, 64>(a, causal, stream);
  if (K == 128 && V == 128) return launch_t<128, 128>(a, causal, stream);
  return hipErrorInvalidValue;
}

}  // namespace memt
