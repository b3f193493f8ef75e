// Inter-chunk state scan of the chunked GDN-2 update: the wide heads
// (d = 256 and d = 512) and the group combine of every width.  d <= 128 runs
// the column-split scan of scan_kernel.hip around the same combine_kernel.
//
// One workgroup (8 waves) per (sequence or chunk group, head, 64-column slice)
// holds a K x 64 slice of the head's fp32 state in MFMA accumulators and walks
// the chunks in order (models/qwen/ops/_triton/state.py:76-115):
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
// use in chunk c (one register buffer), between the MFMAs that consume the
// other fragments; plan entries come from a per-wave cache of 64 chunks.
// Loads past the last chunk reload the last chunk, so every load is
// unconditional and the compiler's vmcnt waits stay exact.  The scan proper
// at d >= 256 takes some records through LDS instead (direct loads, waited for
// by counted vmcnt waits): the chunk's kg^T record and decay row, issued at the
// chunk's start and read in its state update, and at d = 256 also W, two
// buffers a chunk ahead.
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

// d >= 256, the scan proper: the chunk's kg^T record and decay row come through
// LDS (direct loads at the start of the chunk, read in its state update) instead
// of a register buffer a chunk ahead.  At d = 512 that is 96 VGPRs the 64-column
// slice needs to stay within 256 without spilling (commit 3.44 -> 2.93 ms); at
// d = 256 the causal scan's 48 (update step 2550 -> 2419 us).  The transition
// kernels keep the register buffer.
__host__ __device__ constexpr bool scan_kd_lds(int K) { return K > 128; }

template <int K, int NC, bool CAUSAL, bool KDL>
struct ScanFrag {
  static constexpr int KS = K / 32;
  static constexpr int RT = K / 64;    // 16-row state tiles per wave
  static constexpr int CT = NC / 32;   // 16-column tiles per wave (half the columns)
  static constexpr int RTK = KDL ? 1 : RT;
  static constexpr int KSW = (KDL && K == 256) ? 1 : KS;  // d = 256 scan proper: W through LDS
  f16x8 w[KSW];
  f16x8 qg[CAUSAL ? KS : 1];
  f16x8 kg[RTK][2];
  f16x8 aq[CAUSAL ? 2 : 1];
  f16x4 u[CT];
  f32x4 d[RTK];
};

constexpr int kScanThreads = 512;
// Column pitches (in elements) of the f16 LDS tiles: K + kSPad for f16(S),
// 64 + kVPad for f16(V_new), K + kSPad for the combine's bf16 S halves.
constexpr int kSPad = 4;
constexpr int kVPad = 4;

// Groups [first, first + count) of sequence n.
__device__ __forceinline__ void sequence_groups(const int32_t* soff, int n, int L, int& first, int& count) {
  const int lane = threadIdx.x & 63;
  int sum = 0;
  for (int n0 = 0; n0 < n; n0 += 64) {
    const int m = n0 + lane;
    int cnt = 0;
    if (m < n) cnt = (soff[m + 1] - soff[m] + L - 1) / L;
    sum += wave_sum_int(cnt);
  }
  first = sum;
  count = (soff[n + 1] - soff[n] + L - 1) / L;
}

// MODE 0: the scan (per sequence, or per group from its start state), columns of S
// MODE 1: group transition P_g, columns of the K x K identity, no values
// MODE 2: group contribution Q_g, value columns from a zero state
// The workgroup carries NC columns starting at column cbase; its LDS tiles
// hold only those columns.
template <int K, int V, int NC, bool CAUSAL, int MODE>
__device__ __forceinline__ void scan_body(const StateArgs& a, int unitg, int h, int cbase, _Float16* S_lds,
                                          _Float16* Vn_lds, char* kd_lds = nullptr, char* w_lds = nullptr) {
  constexpr bool KD_LDS = scan_kd_lds(K) && MODE == 0;
  // d = 256, the scan proper: W through two LDS buffers, a chunk ahead
  constexpr bool W_LDS = KD_LDS && K == 256;
  constexpr int WBYTES = kChunk * K * 2, W_PER_WAVE = WBYTES / 1024 / (kScanThreads / 64);
  using F = ScanFrag<K, NC, CAUSAL, KD_LDS>;
  constexpr int C = kChunk;
  constexpr int KS = F::KS, RT = F::RT, CT = F::CT;
  // Up to d = 128 all f16(S) operands of a chunk (16 at most) are read from LDS
  // in one batch before the chunk's MFMAs; the wider slices keep one read per
  // step, interleaved by the compiler (their registers are fuller, and batching
  // there measured slower).
  constexpr bool BATCH = K <= 128 && KS * CT <= 16;
  constexpr int SKP = K + kSPad;  // pitch of column-major f16(S)
  constexpr int VNP = C + kVPad;  // pitch of column-major f16(V_new)
  static_assert(MODE == 0 || !CAUSAL, "the transition modes write no output");
  static_assert(RT >= 1 && CT >= 1, "tile shape");
  const int H = a.H;

  int c_begin, c_end, seq = unitg;
  bool first = true, last = true;
  if (a.group_L == 0) {
    c_begin = a.seq_chunk_offsets[seq];
    c_end = a.seq_chunk_offsets[seq + 1];
  } else {
    const GroupLoc gl = locate_group(a.seq_chunk_offsets, a.n_seq, a.group_L, unitg);
    if (!gl.valid) return;
    seq = __builtin_amdgcn_readfirstlane(gl.seq);
    c_begin = __builtin_amdgcn_readfirstlane(gl.c_begin);
    c_end = __builtin_amdgcn_readfirstlane(gl.c_end);
    const int g_first = __builtin_amdgcn_readfirstlane(gl.first_group);
    const int g_count = __builtin_amdgcn_readfirstlane(gl.n_groups);
    first = unitg == g_first;
    last = unitg + 1 == g_first + g_count;
    if (MODE != 0 && last) return;  // the last group's transition is never used
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = w & 3, half = w >> 2;
  const int lr = lane & 15, lg = lane >> 4;
  const int lcol0 = half * (NC / 2);  // first column of this wave in the LDS tiles
  const int col0 = cbase + lcol0;     // and in the state

  // The starting state of this workgroup's slice, tile (rt, ct): rows
  // 16 (q RT + rt) + 4 lg + e, column col0 + 16 ct + lr.  Every group of a
  // multi-group sequence starts from the combine's S0 (the first one from the
  // combine's copy of h0), so when ht and h0 name the same slot the last
  // group's ht write cannot overtake the first group's h0 read.
  const bool from_s0 = MODE == 0 && !(first && last);
  const float* s0 = a.grp.S0 + ((size_t)unitg * H + h) * K * V;  // C-frag order (from_s0)
  const int slot = (!from_s0 && a.h0_slot) ? a.h0_slot[seq] : seq;
  const float* h0p = (MODE == 0 && a.h0 != nullptr) ? a.h0 + ((size_t)slot * H + h) * K * V : nullptr;
  auto start_tile = [&](int rt, int ct) {
    if (from_s0)
      return *(const f32x4*)(s0 + ((size_t)((q * RT + rt) * (V / 16) + (col0 >> 4) + ct) * 64 + lane) * 4);
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = 16 * (q * RT + rt) + 4 * lg + e;
      const int col = col0 + 16 * ct + lr;
      if constexpr (MODE == 1) r[e] = row == col ? 1.f : 0.f;
      else r[e] = h0p ? h0p[(size_t)row * V + col] : 0.f;
    }
    return r;
  };

  // channel pass of this workgroup's value columns (d = 512: two passes of 256)
  constexpr int NPU = wy_passes(K);
  const int pu = NPU > 1 ? col0 / (V / NPU) : 0;
  // Value exponent of this workgroup's columns: the largest of its chunks' U
  // exponents and of its starting state's, so that U * 2^-ew and S * 2^-ew
  // stay inside the f16 operand range.  The columns of S are independent, so
  // every workgroup may use its own.  The transition (MODE 1) is scale-free.
  // It is formed before the state is held (the starting slice is read once for
  // its max, then again as the state), which keeps the register peak of the
  // widest slices where it was.
  int ew = 0;
  if constexpr (MODE != 1) {
    int eu = 0;
    for (int c0 = c_begin; c0 < c_end; c0 += 64) {
      const int c = c0 + lane;
      if (c < c_end) eu = max(eu, a.in.uexp[((size_t)c * H + h) * NPU + pu]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) eu = max(eu, __shfl_xor(eu, off, 64));
    float smax = 0.f;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const f32x4 x = start_tile(rt, ct);
#pragma unroll
        for (int e = 0; e < 4; ++e) smax = fmaxf(smax, fabsf(x[e]));
      }
    smax = wave_max(smax);
    float* red = (float*)Vn_lds;  // free until the first chunk's V_new
    if (lane == 0) red[w] = smax;
    lds_barrier();
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < kScanThreads / 64; ++i) m = fmaxf(m, red[i]);
    ew = __builtin_amdgcn_readfirstlane(max(eu, value_exponent(m)));
  }
  const float oscale = pow2_exact(ew);  // back to the values' own scale on store
  const float iscale = pow2_exact(-ew);

  f32x4 S[RT][CT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      S[rt][ct] = start_tile(rt, ct);
      if constexpr (MODE != 1) S[rt][ct] *= iscale;
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
        *(f16x4*)(&S_lds[(lcol0 + 16 * ct + lr) * SKP + 16 * (q * RT + rt) + 4 * lg]) = b4;
      }
  };

  // Plan entries of chunks [mbase, mbase + 64), one chunk per lane, read out
  // with readlane.  Loading them per chunk would make the compiler move each
  // entry to a scalar register right after its load, waiting for every
  // outstanding prefetch; this way the wait comes once per 64 chunks.
  int mbase = c_begin - 64;
  // The chunk's U exponent rides in bits 8.. of the cached flags (the flags use
  // bits 0-1), so it costs no register of its own.
  int m_flags = 0, m_block = -1, m_tok0 = 0, m_len = 0;
  int flags = 0, block = -1, tok0 = 0, len = 0;
  auto meta = [&](int c) {
    if (c - mbase >= 64) {
      mbase = c;
      const int cc = c + lane;
      const bool ok = cc < c_end;
      m_flags = !ok ? 0 : a.chunk_flags ? a.chunk_flags[cc] : MEMT_GDN2_CHUNK_COMMIT;
      if constexpr (MODE != 1) m_flags |= (ok ? a.in.uexp[((size_t)cc * H + h) * NPU + pu] : 0) << 8;
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
  // Record fragments, each (re)loaded right after its last use: the loads of
  // chunk c + 1 spread over chunk c's MFMAs instead of queueing in bursts.
  auto load_w = [&](int c, int s) {
    const size_t fo = ((size_t)c * H + h) * (size_t)(C * K) + ((size_t)(q * KS + s) * 64 + lane) * 8;
    if constexpr (!W_LDS) f.w[s] = *(const f16x8*)(a.in.W + fo);
    if constexpr (CAUSAL) f.qg[s] = *(const f16x8*)(a.in.qg + fo);
  };
  auto stage_w = [&](int c, int b) {
    if constexpr (W_LDS) {
      const char* src = (const char*)(a.in.W + ((size_t)c * H + h) * (size_t)(C * K));
#pragma unroll
      for (int i = 0; i < W_PER_WAVE; ++i) {
        const int fr = w * W_PER_WAVE + i;
        lds_dma16(src + (size_t)fr * 1024 + 16 * lane, w_lds + b * WBYTES + fr * 1024);
      }
    }
  };
  auto load_u = [&](int c) {
    if constexpr (MODE != 1) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        f.u[ct] = *(const f16x4*)(a.in.U + ((size_t)c * H + h) * (size_t)(C * V) +
                                  ((size_t)(q * (V / 16) + (col0 >> 4) + ct) * 64 + lane) * 4);
    } else {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) f.u[ct] = f16x4{};
    }
  };
  auto load_aq = [&](int c) {
    if constexpr (CAUSAL) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
        f.aq[s] = *(const f16x8*)(a.in.Aqk + ((size_t)c * H + h) * (size_t)(C * C) +
                                  ((size_t)(q * 2 + s) * 64 + lane) * 8);
    }
  };
  auto load_kd = [&](int c, int rt) {
    if constexpr (!KD_LDS) {
      const size_t unit = (size_t)c * H + h;
      const int rtile = q * RT + rt;
      f.d[rt] = *(const f32x4*)(a.in.decay + unit * K + 16 * rtile + 4 * lg);
#pragma unroll
      for (int s = 0; s < 2; ++s)
        f.kg[rt][s] = *(const f16x8*)(a.in.kgT + unit * (size_t)(C * K) + ((size_t)(rtile * 2 + s) * 64 + lane) * 8);
    }
  };
  // KD_LDS: chunk c's kg^T record (C K halves, 2 K / 16 fragments of 1 KiB) and decay
  // row (K floats) into kd_lds by direct loads, the fragments split over the 8 waves,
  // the decay row's K / 256 KiB on wave 0 (which issues that many more)
  constexpr int KD_FRAG = 2 * K / 16, KD_PER_WAVE = KD_FRAG / (kScanThreads / 64), KD_DEC = K * 4 / 1024;
  auto stage_kd = [&](int c) {
    if constexpr (KD_LDS) {
      const size_t unit = (size_t)c * H + h;
      const char* kg_src = (const char*)(a.in.kgT + unit * (size_t)(C * K));
#pragma unroll
      for (int i = 0; i < KD_PER_WAVE; ++i) {
        const int fr = w * KD_PER_WAVE + i;
        lds_dma16(kg_src + (size_t)fr * 1024 + 16 * lane, kd_lds + fr * 1024);
      }
      if (w == 0) {
        const char* d_src = (const char*)(a.in.decay + unit * K);
#pragma unroll
        for (int i = 0; i < KD_DEC; ++i) lds_dma16(d_src + i * 1024 + 16 * lane, kd_lds + KD_FRAG * 1024 + i * 1024);
      }
    }
  };
  // the first chunk's fragments, in the order the loop consumes and reloads them,
  // so that its vmcnt waits stay partial from the first iteration on
  auto load_all = [&](int c) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      load_w(c, s);
      asm volatile("" ::: "memory");
    }
    load_u(c);
    asm volatile("" ::: "memory");
    load_aq(c);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      load_kd(c, rt);
      asm volatile("" ::: "memory");
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
    stage_w(c_begin, 0);
    load_all(c_begin);
    if constexpr (W_LDS) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      lds_barrier();  // the first chunk's W is in LDS
    }
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
                a.snaps[soff + (size_t)row * V + col0 + 16 * ct + lr] = S[rt][ct][e] * oscale;
              }
        }
      }
      const int cur_flags = flags, cur_tok0 = tok0, cur_len = len;
      // this chunk's U to the workgroup's scale, 2^(uexp - ew) <= 1, formed in scalar registers
      const float uscale = pow2_exact((cur_flags >> 8) - ew);
      meta(cn);
      stage_kd(c);  // KD_LDS: this chunk's kg^T and decay, landed by its state update
      stage_w(cn, (c - c_begin + 1) & 1);  // W_LDS: the next chunk's W into the other buffer
      const char* const wcur =
          W_LDS ? w_lds + ((c - c_begin) & 1) * WBYTES + ((size_t)(q * KS) * 64 + lane) * 16 : nullptr;
      // ---- V_new (token rows 16 q .. 16 q + 15) and o^T from f16(S) ----
      f32x4 acc[CT], acco[CAUSAL ? CT : 1];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        acc[ct] = zero4();
        if constexpr (CAUSAL) acco[ct] = zero4();
      }
      if constexpr (BATCH) {
        // every f16(S) operand read ahead of the MFMAs (the scheduling barrier
        // keeps the compiler from pairing each read with its own wait), so the
        // chunk pays one LDS latency instead of one per operand
        f16x8 sb[KS][CT];
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) sb[s][ct] = b_operand(S_lds, SKP, lcol0 + 16 * ct + lr, s);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            acc[ct] = mfma_f16(f.w[s], sb[s][ct], acc[ct]);
            if constexpr (CAUSAL) acco[ct] = mfma_f16(sb[s][ct], f.qg[s], acco[ct]);
          }
          load_w(cn, s);  // W and qg of the next chunk, step s
        }
      } else {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            const f16x8 sb = b_operand(S_lds, SKP, lcol0 + 16 * ct + lr, s);
            f16x8 wv;
            if constexpr (W_LDS) wv = *(const f16x8*)(wcur + s * 1024);
            else wv = f.w[s];
            acc[ct] = mfma_f16(wv, sb, acc[ct]);
            if constexpr (CAUSAL) acco[ct] = mfma_f16(sb, f.qg[s], acco[ct]);
          }
          load_w(cn, s);  // W and qg of the next chunk, step s
        }
      }
      f16x4 un[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) un[ct] = f.u[ct];
      load_u(cn);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        f16x4 vn;
#pragma unroll
        for (int e = 0; e < 4; ++e) vn[e] = (_Float16)((float)un[ct][e] * uscale - acc[ct][e]);
        *(f16x4*)(&Vn_lds[(lcol0 + 16 * ct + lr) * VNP + 16 * q + 4 * lg]) = vn;
      }
      if constexpr (KD_LDS) {
        // at most the next chunk's W and qg prefetches issued since are left in
        // flight (one per step each; loads complete in issue order), so this
        // chunk's direct loads have landed; the U prefetches issued after them are
        // waited for too (leaving those two in flight as well measured the same)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(W_LDS ? W_PER_WAVE + (CAUSAL ? KS : 0) : CAUSAL ? 2 * KS : KS)
                     : "memory");
      }
      lds_barrier();

      // ---- causal output; S = decay * S + kg^T . V_new ----
      f16x8 vb[CT][2];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int s = 0; s < 2; ++s) vb[ct][s] = b_operand(Vn_lds, VNP, lcol0 + 16 * ct + lr, s);
      if constexpr (CAUSAL) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
          for (int e = 0; e < 4; ++e) acco[ct][e] *= a.scale;
#pragma unroll
          for (int s = 0; s < 2; ++s) acco[ct] = mfma_f16(vb[ct][s], f.aq[s], acco[ct]);
        }
        load_aq(cn);
      }
      const bool commit = (cur_flags & MEMT_GDN2_CHUNK_COMMIT) != 0;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        if constexpr (KD_LDS) {
          if (commit) {
            const int rtile = q * RT + rt;
            const f32x4 dv = *(const f32x4*)(kd_lds + KD_FRAG * 1024 + (16 * rtile + 4 * lg) * 4);
            f16x8 kg2[2];
#pragma unroll
            for (int s = 0; s < 2; ++s) kg2[s] = *(const f16x8*)(kd_lds + (rtile * 2 + s) * 1024 + 16 * lane);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
              for (int e = 0; e < 4; ++e) S[rt][ct][e] *= dv[e];
#pragma unroll
              for (int s = 0; s < 2; ++s) S[rt][ct] = mfma_f16(kg2[s], vb[ct][s], S[rt][ct]);
            }
          }
        } else {
          if (commit) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
              for (int e = 0; e < 4; ++e) S[rt][ct][e] *= f.d[rt][e];
#pragma unroll
              for (int s = 0; s < 2; ++s) S[rt][ct] = mfma_f16(f.kg[rt][s], vb[ct][s], S[rt][ct]);
            }
          }
          load_kd(cn, rt);  // decay and kg^T rows of the next chunk
        }
      }
      if constexpr (CAUSAL) {
        // lane holds o[16 q + lr][col0 + 16 ct + 4 lg + e]
        const int t = 16 * q + lr;
        if (t < cur_len) {
          __bf16* orow = a.o + ((size_t)(cur_tok0 + t) * H + h) * V + col0 + 4 * lg;
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            bf16x4 o4;
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = (__bf16)(acco[ct][e] * oscale);
            *(bf16x4*)(orow + 16 * ct) = o4;
          }
        }
      }
      if constexpr (W_LDS) {
        // the next chunk's W (issued at this chunk's start) has landed: only the
        // qg prefetches (one per step) issued after it may still be in flight
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CAUSAL ? KS : 0) : "memory");
      }
      write_S_lds();
      lds_barrier();
    }
  }

  if constexpr (MODE == 1) {
    // P_g split into bf16 hi + lo, in A-frag order (rows = P rows, reduction = P
    // columns): the A operands of the combine, one contiguous 16-byte load per lane
    const size_t base = ((size_t)unitg * H + h) * K * K;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const size_t idx = base + afrag_index(16 * (q * RT + rt) + 4 * lg + e, col0 + 16 * ct + lr, K);
          const __bf16 hi = (__bf16)S[rt][ct][e];
          a.grp.P_hi[idx] = hi;
          a.grp.P_lo[idx] = (__bf16)(S[rt][ct][e] - (float)hi);
        }
  } else if constexpr (MODE == 2) {
    float* qo = a.grp.Q + ((size_t)unitg * H + h) * K * V;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        *(f32x4*)(qo + ((size_t)((q * RT + rt) * (V / 16) + (col0 >> 4) + ct) * 64 + lane) * 4) = S[rt][ct] * oscale;
  } else if (last && a.ht != nullptr) {
    float* out = a.ht + ((size_t)(a.ht_slot ? a.ht_slot[seq] : seq) * H + h) * K * V;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = 16 * (q * RT + rt) + 4 * lg + e;
          out[(size_t)row * V + col0 + 16 * ct + lr] = S[rt][ct][e] * oscale;
        }
  }
}

// Blocks are (slice, unit, head) with the slice outermost: with units * H a
// multiple of 8 the slices of one (unit, head), which read the same chunk
// records, land on the same XCD (blocks go to XCDs round-robin).
template <int K, int V, bool CAUSAL>
__global__ __launch_bounds__(kScanThreads) void state_kernel(StateArgs a, int units) {
  constexpr int NS = scan_slice(V);
  __shared__ __attribute__((aligned(16))) _Float16 S_lds[NS * (K + kSPad)];
  __shared__ __attribute__((aligned(16))) _Float16 Vn_lds[NS * (kChunk + kVPad)];
  __shared__ __attribute__((aligned(1024))) char kd_lds[scan_kd_lds(K) ? 2 * kChunk * K + 4 * K : 16];
  __shared__ __attribute__((aligned(1024))) char w_lds[K == 256 ? 2 * 2 * kChunk * K : 16];
  const int per = units * a.H, b = blockIdx.x % per;
  scan_body<K, V, NS, CAUSAL, 0>(a, b / a.H, b % a.H, NS * (blockIdx.x / per), S_lds, Vn_lds, kd_lds, w_lds);
}

// Phase 1 of the two-level scan: nP = (K / slice) units H blocks form P_g and
// as many form Q_g.  The P and Q blocks of one (group, head, slice) read the
// same W and kg^T records, so they are interleaved in runs of 8 (blocks b and
// b + 8 of every 16): the pair shares an XCD and its L2 and runs at the same
// time.
template <int K, int V>
__global__ __launch_bounds__(kScanThreads) void trans_kernel(StateArgs a, int units) {
  constexpr int NSK = scan_slice(K), NSV = scan_slice(V);
  constexpr int NCM = NSK > NSV ? NSK : NSV;
  static_assert(K / NSK == V / NSV, "as many P as Q blocks");
  __shared__ __attribute__((aligned(16))) _Float16 S_lds[NCM * (K + kSPad)];
  __shared__ __attribute__((aligned(16))) _Float16 Vn_lds[NCM * (kChunk + kVPad)];
  const int per = units * a.H, nP = per * (K / NSK);
  bool is_p;
  int b;
  if (nP % 8 == 0) {
    is_p = ((blockIdx.x >> 3) & 1) == 0;
    b = (blockIdx.x >> 4) * 8 + (blockIdx.x & 7);
  } else {
    is_p = (int)blockIdx.x < nP;
    b = is_p ? blockIdx.x : blockIdx.x - nP;
  }
  const int r = b % per, slice = b / per;
  if (is_p)
    scan_body<K, V, NSK, false, 1>(a, r / a.H, r % a.H, NSK * slice, S_lds, Vn_lds);
  else
    scan_body<K, V, NSV, false, 2>(a, r / a.H, r % a.H, NSV * slice, S_lds, Vn_lds);
}

// Phase 2 of the two-level scan, one workgroup per (sequence, head, 16 state
// columns): S_{g+1} = P_g S_g + Q_g over the sequence's groups, writing the state
// entering every group but the first.  P_g S_g is split-bf16 MFMA
// (P_hi S_hi + P_hi S_lo + P_lo S_hi) with fp32 accumulation; P and Q of the
// next group are prefetched while the current one is applied.
template <int K, int V>
struct CombineFrag {
  static constexpr int RT = K / 64, KS = K / 32;
  bf16x8 ph[RT][KS], pl[RT][KS];
  f32x4 q[RT][1];
};

template <int K, int V>
__global__ __launch_bounds__(256) void combine_kernel(StateArgs a) {
  using F = CombineFrag<K, V>;
  constexpr int BV = 16, NV = V / BV, RT = F::RT, KS = F::KS, CT = 1, SP = K + kSPad;
  __shared__ __attribute__((aligned(16))) __bf16 Shi[BV * SP];
  __shared__ __attribute__((aligned(16))) __bf16 Slo[BV * SP];
  const int H = a.H;
  // XCD-aware order: the NV column slices of one (sequence, head) read the same
  // P_g and Q_g, so they share an XCD (and its L2); blocks are dispatched to
  // XCDs round-robin by block index.
  const int total = gridDim.x;
  int bid = blockIdx.x;
  if ((total & 7) == 0) bid = (blockIdx.x & 7) * (total >> 3) + (blockIdx.x >> 3);
  const int vs = bid % NV, h = (bid / NV) % H, n = bid / (NV * H);
  int g0, gcount;
  sequence_groups(a.seq_chunk_offsets, n, a.group_L, g0, gcount);
  g0 = __builtin_amdgcn_readfirstlane(g0);
  gcount = __builtin_amdgcn_readfirstlane(gcount);
  if (gcount <= 1) return;
  const int g1 = g0 + gcount;
  const int v0 = vs * BV, tid = threadIdx.x, w = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;

  f32x4 S[RT][CT];
  const float* h0p = a.h0 ? a.h0 + ((size_t)(a.h0_slot ? a.h0_slot[n] : n) * H + h) * K * V : nullptr;
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
  {
    // the first group's start state: the scan reads it here, never from h0
    float* S0 = a.grp.S0 + ((size_t)g0 * H + h) * K * V;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        *(f32x4*)(S0 + ((size_t)((w * RT + rt) * (V / 16) + (v0 >> 4) + ct) * 64 + lane) * 4) = S[rt][ct];
  }

  // First load, in the order the loop consumes and reloads the fragments: the
  // empty asm statements keep the compiler from reordering the loads, so the
  // loop's vmcnt waits stay partial on its entry path too.
  auto load = [&](int g, F& f) {
    const size_t pb = ((size_t)g * H + h) * K * K;
    const float* Q = a.grp.Q + ((size_t)g * H + h) * K * V;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const size_t fo = pb + ((size_t)((w * RT + rt) * KS + s) * 64 + lane) * 8;
        f.ph[rt][s] = *(const bf16x8*)(a.grp.P_hi + fo);
        f.pl[rt][s] = *(const bf16x8*)(a.grp.P_lo + fo);
        asm volatile("" ::: "memory");
      }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        f.q[rt][ct] = *(const f32x4*)(Q + ((size_t)((w * RT + rt) * (V / 16) + (v0 >> 4) + ct) * 64 + lane) * 4);
  };
  // One step applies group g from f, reloading each fragment of f for group
  // gload right after its last use, so the loads spread over the MFMAs and the
  // rest of the step.
  auto step = [&](int g, F& f, int gload) {
    const size_t pb = ((size_t)gload * H + h) * K * K;
    const float* Qn = a.grp.Q + ((size_t)gload * H + h) * K * V;
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
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          acc[rt][ct] = mfma_bf16(f.ph[rt][s], bh[ct], acc[rt][ct]);
          acc[rt][ct] = mfma_bf16(f.ph[rt][s], bl[ct], acc[rt][ct]);
          acc[rt][ct] = mfma_bf16(f.pl[rt][s], bh[ct], acc[rt][ct]);
        }
        const size_t fo = pb + ((size_t)((w * RT + rt) * KS + s) * 64 + lane) * 8;
        f.ph[rt][s] = *(const bf16x8*)(a.grp.P_hi + fo);
        f.pl[rt][s] = *(const bf16x8*)(a.grp.P_lo + fo);
      }
    }
    float* S0 = a.grp.S0 + ((size_t)(g + 1) * H + h) * K * V;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const size_t qo = ((size_t)((w * RT + rt) * (V / 16) + (v0 >> 4) + ct) * 64 + lane) * 4;
        S[rt][ct] = acc[rt][ct] + f.q[rt][ct];
        *(f32x4*)(S0 + qo) = S[rt][ct];
        f.q[rt][ct] = *(const f32x4*)(Qn + qo);
      }
    lds_barrier();
  };
  // groups g0 .. g1 - 2 each produce the start state of the next group
  const int glast = g1 - 2;
  F f;
  load(g0, f);
  for (int g = g0; g <= glast; ++g) step(g, f, min(g + 1, glast));
}

template <int K, int V>
hipError_t launch_t(const StateArgs& a, bool causal, hipStream_t stream) {
  if constexpr (K > 256) {
    // d = 512: the plain scan without the causal output (the final-state and
    // snapshot-read modes of the wide-state model)
    if (causal || a.group_L > 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL((state_kernel<K, V, false>), dim3(a.n_seq * a.H * (V / scan_slice(V))), dim3(kScanThreads),
                       0, stream, a, a.n_seq);
    return hipGetLastError();
  } else if constexpr (K <= 128) {
    // d <= 128: the column-split scan (scan_kernel.hip) around the same combine
    int units = a.n_seq;
    if (a.group_L > 0) {
      units = group_bound(a.n_chunk, a.n_seq, a.group_L);
      const hipError_t e = launch_colscan(a, K, V, false, 1, units, stream);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((combine_kernel<K, V>), dim3((V / 16) * a.H * a.n_seq), dim3(256), 0, stream, a);
    }
    return launch_colscan(a, K, V, causal, 0, units, stream);
  } else {
    int units = a.n_seq;
    if (a.group_L > 0) {
      units = group_bound(a.n_chunk, a.n_seq, a.group_L);
      const int nt = units * a.H * (K / scan_slice(K) + V / scan_slice(V));
      hipLaunchKernelGGL((trans_kernel<K, V>), dim3(nt), dim3(kScanThreads), 0, stream, a, units);
      hipLaunchKernelGGL((combine_kernel<K, V>), dim3((V / 16) * a.H * a.n_seq), dim3(256), 0, stream, a);
    }
    const dim3 grid(units * a.H * (V / scan_slice(V))), block(kScanThreads);
    if (causal)
      hipLaunchKernelGGL((state_kernel<K, V, true>), grid, block, 0, stream, a, units);
    else
      hipLaunchKernelGGL((state_kernel<K, V, false>), grid, block, 0, stream, a, units);
    return hipGetLastError();
  }
}

}  // namespace

hipError_t launch_state(const StateArgs& a, int K, int V, bool causal, hipStream_t stream) {
  if (a.n_seq == 0) return hipSuccess;
  if (K == 64 && V == 64) return launch_t<64, 64>(a, causal, stream);
  if (K == 128 && V == 128) return launch_t<128, 128>(a, causal, stream);
  if (K == 256 && V == 256) return launch_t<256, 256>(a, causal, stream);
  if (K == 512 && V == 512) return launch_t<512, 512>(a, causal, stream);
  return hipErrorInvalidValue;
}

}  // namespace memt
