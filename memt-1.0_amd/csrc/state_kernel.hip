// Inter-chunk state scan of the chunked GDN-2 update.
//
// One workgroup (4 waves) per (sequence, head, slice of BV state columns).
// Columns of the state are independent in the recurrence (v_new[:, j] only
// depends on S[:, j]), so each workgroup keeps its K x BV fp32 slice of S in
// MFMA accumulators for the whole sequence and walks the chunks in order
// (models/qwen/ops/_triton/state.py:76-115):
//
//   snapshot S if the chunk starts a read block
//   V_new = U - W . f16(S)                         (erase path)
//   o     = scale * qg . f16(S) + Aqk . V_new       (causal output, optional)
//   S     = decay * S + kg^T . f16(V_new)           (value path, if committed)
// Every product is fp16 MFMA with fp32 accumulation; S stays fp32.
//
// Wave w owns S rows [w*K/4, (w+1)*K/4) and V_new / o token rows [16w, 16w+16),
// so it reads only its quarter of each chunk record.  f16(S) and f16(V_new)
// cross waves through two column-major LDS tiles, with two LDS-only barriers
// per chunk.  The W / qg / kg^T / Aqk records are P-frags, whose reduction
// index pairs with B operands gathered as two 8-byte LDS reads per lane.
//
// Prefetch: everything a chunk needs from global memory (its operand
// fragments and its plan entries) is loaded into registers two chunks ahead;
// the loop is unrolled by two so the two register buffers alternate without
// copies, and the compiler's vmcnt waits stay exact.
//
// Long sequences use a two-level scan over groups of chunks (the recurrence is
// linear in S): the same kernel first runs on [I | 0] per group to form the
// group transition P_g and its zero-start contribution Q_g (modes 1 and 2),
// combine_kernel then chains S_{g+1} = P_g S_g + Q_g per sequence (split-bf16
// MFMA, ~2^-16 relative), and the scan proper runs per group from S_g.
#include "gdn2_internal.h"

namespace memt {
namespace {

template <int K, int V, int BV, bool CAUSAL>
struct ScanFrag {
  static constexpr int KS = K / 32;
  static constexpr int RT = K / 64;   // 16-row S tiles per wave
  static constexpr int CT = BV / 16;  // 16-column tiles per workgroup
  f16x8 w[KS];
  f16x8 qg[CAUSAL ? KS : 1];
  f16x8 kg[RT][2];
  f16x8 aq[CAUSAL ? 2 : 1];
  f16x4 u[CT];
  f32x4 d[RT];
  int flags, block, tok0, len;
};

// MODE 0: the scan (per sequence, or per group from its start state)
// MODE 1: group transition P_g, columns of the K x K identity, no values
// MODE 2: group contribution Q_g, value columns from a zero state
template <int K, int V, int BV, bool CAUSAL, int MODE>
__global__ __launch_bounds__(256) void state_kernel(StateArgs a) {
  using F = ScanFrag<K, V, BV, CAUSAL>;
  constexpr int C = kChunk;
  constexpr int NC = MODE == 1 ? K : V;  // state columns of this mode
  constexpr int NV = NC / BV;
  static_assert(MODE == 0 || !CAUSAL, "the transition modes write no output");
  constexpr int KS = F::KS;
  constexpr int RT = F::RT;
  constexpr int CT = F::CT;
  constexpr int SKP = K + 8;  // pitch of column-major f16(S)
  constexpr int VNP = C + 8;  // pitch of column-major f16(V_new)
  static_assert(RT >= 1 && CT >= 1, "tile shape");

  __shared__ __attribute__((aligned(16))) _Float16 S_lds[BV * SKP];
  __shared__ __attribute__((aligned(16))) _Float16 Vn_lds[BV * VNP];

  // XCD-aware order: the NV slices of one (sequence, head) share an XCD (and its L2),
  // since they all read the same per-chunk records.
  const int total = gridDim.x;
  int bid = blockIdx.x;
  if ((total & 7) == 0) bid = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int vs = bid % NV;
  const int h = (bid / NV) % a.H;
  const int unitg = bid / (NV * a.H);  // sequence, or group when grouped
  const int H = a.H;
  const int v0 = vs * BV;  // first state column (of P for MODE 1, of V otherwise)

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

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  // S tile rt of this wave: rows 16*(w*RT + rt) + 4*lg + e, column v0 + 16*ct + lr
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
        const int row = 16 * (w * RT + rt) + 4 * lg + e;
        const int col = v0 + 16 * ct + lr;
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
        *(f16x4*)(&S_lds[(16 * ct + lr) * SKP + 16 * (w * RT + rt) + 4 * lg]) = b4;
      }
  };

  // Plan entries of chunks [mbase, mbase + 64), one chunk per lane, read out
  // with readlane.  Loading them per chunk would make the compiler move each
  // entry to a scalar register right after its load, waiting for every
  // outstanding prefetch; this way the wait comes once per 64 chunks.
  int mbase = c_begin - 64;
  int m_flags = 0, m_block = -1, m_tok0 = 0, m_len = 0;
  auto meta = [&](int c, F& f) {
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
    f.flags = __builtin_amdgcn_readlane(m_flags, i);
    f.block = __builtin_amdgcn_readlane(m_block, i);
    f.tok0 = CAUSAL ? __builtin_amdgcn_readlane(m_tok0, i) : 0;
    f.len = CAUSAL ? __builtin_amdgcn_readlane(m_len, i) : 0;
  };

  auto load = [&](int c, F& f) {
    meta(c, f);
    const size_t unit = (size_t)c * H + h;
    const _Float16* Wp = a.in.W + unit * (size_t)(C * K);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const size_t fo = ((size_t)(w * KS + s) * 64 + lane) * 8;
      f.w[s] = *(const f16x8*)(Wp + fo);
      if constexpr (CAUSAL) f.qg[s] = *(const f16x8*)(a.in.qg + unit * (size_t)(C * K) + fo);
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
    if constexpr (MODE != 1) {
      const _Float16* Up = a.in.U + unit * (size_t)(C * V);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        f.u[ct] = *(const f16x4*)(Up + ((size_t)(w * (V / 16) + (v0 >> 4) + ct) * 64 + lane) * 4);
    } else {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) f.u[ct] = f16x4{};
    }
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
        const f16x8 sb = b_operand(S_lds, SKP, ct, s);
        acc[ct] = mfma_f16(f.w[s], sb, acc[ct]);
        if constexpr (CAUSAL) acco[ct] = mfma_f16(f.qg[s], sb, acco[ct]);
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
          const int row = 16 * (w * RT + rt) + 4 * lg + e;
          out[(size_t)row * NC + v0 + 16 * ct + lr] = S[rt][ct][e];
        }
  }
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

template <int K, int V, int BV>
hipError_t launch_t(const StateArgs& a, bool causal, hipStream_t stream) {
  const dim3 block(256);
  int units = a.n_seq;
  if (a.group_L > 0) {
    units = group_bound(a.n_chunk, a.n_seq, a.group_L);
    hipLaunchKernelGGL(group_table_kernel, dim3(1), block, 0, stream, a.seq_chunk_offsets, a.n_seq, a.group_L,
                       a.grp.seq_group_offsets, a.grp.group_chunk_offsets, a.grp.group_seq);
    hipLaunchKernelGGL((state_kernel<K, V, BV, false, 1>), dim3((K / BV) * a.H * units), block, 0, stream, a);
    hipLaunchKernelGGL((state_kernel<K, V, BV, false, 2>), dim3((V / BV) * a.H * units), block, 0, stream, a);
    hipLaunchKernelGGL((combine_kernel<K, V>), dim3((V / 32) * a.H * a.n_seq), block, 0, stream, a);
  }
  const dim3 grid((V / BV) * a.H * units);
  if (causal)
    hipLaunchKernelGGL((state_kernel<K, V, BV, true, 0>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((state_kernel<K, V, BV, false, 0>), grid, block, 0, stream, a);
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
