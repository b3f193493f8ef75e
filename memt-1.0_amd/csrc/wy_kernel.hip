// WY stage of the chunked GDN-2 update, one workgroup per (chunk, head).
//
// For a chunk of C <= 64 tokens (rows past the chunk end are zero padded):
//   gk    = 1/ln2 * cumsum_chunk(g)                       (FLA/ops/utils/cumsum.py:116-133)
//   L     = strictly lower, L[i,j] = sum_c (b k)_ic k_jc 2^(gk_ic - gk_jc)
//                                                          (FLA/ops/gdn2/chunk_intra_token_parallel.py:111-123,
//                                                           FLA/ops/gdn2/chunk_intra.py:233-299)
//   A     = (I + L)^-1                                     (chunk_intra.py:326-395)
//   W     = A (b k 2^gk),  U = A (beta v)                  (FLA/ops/gdn2/wy_fast.py:92-142)
//   kg    = k 2^(gk_last - gk), decay = 2^gk_last          (wy_fast.py:125-139)
//   Aqk   = scale * sum_c q_ic k_jc 2^(gk_ic - gk_jc), j <= i, qg = q 2^gk   (causal output only)
// Outputs go to the workspace as MFMA operand fragments of the state scan
// (P-frags for W, qg, kg^T and Aqk; a C-frag for U).
//
// Register layout.  The workgroup has one or two channel groups of 4 waves;
// wave w of a group owns tokens [16w, 16w+16) over the group's channels.  Lane
// l holds token 16w + l%16 and, for channel step s, the 8 channels
//   slot j -> channel c0 + 32 s + 16 (j / 4) + 4 (l / 16) + j % 4      (P-frag order, d <= 128)
//   slot j -> channel c0 + 32 s + 8 (l / 16) + j                       (natural order, d >= 256)
// of every per-token input, c0 the group's first channel.  Loaded once in that
// order, the registers serve directly as MFMA A operands of row-block products
// (any channel order is a valid reduction order) and as B operands of the
// transposed products.  In P-frag order they are also the qg record's fragments
// as they stand; the natural order reads each bf16 row piece with one 16-byte
// load (64 contiguous bytes per row and instruction instead of 32) and permutes
// qg to P-frag order through LDS.  At d >= 256 one workgroup runs per CU and its
// load phase is not hidden behind another's compute, so the wider loads pay
// (an update step at 64 heads, 16384 tokens, d = 256: 2641 -> 2532 us); at
// d = 128 they measured slower (their extra registers spill).
//
// Steps:
//   cumsum    16-lane DPP row scans inside each 16-token block, block totals through LDS.
//   factors   fa = 2^(gk - gk_start) <= 1 and 1/fa, with gk_start the cumulative decay at
//             the first token of the lane's block; per-channel block factors in LDS.
//   L, Aqk    16x16 tiles, computed transposed so that each lane holds one row.
//             Diagonal tiles: fp32 MFMA of (b k fa) and (k / fa), exact products in
//             fp32 range.  Off-diagonal tiles
//             (J < I): fp16 MFMA of (b k fa) and k 2^(gk_start(I) - gk) <= 1, the latter
//             built by wave J.  A block whose in-block decay exceeds 2^96 forms its
//             diagonal tile from exact pairwise factors instead (wave-local shuffles).
//   inverse   A_II by row-wise substitution (fp32), then
//             A_IJ = -A_II sum_{J<=M<I} L_IM A_MJ with fp32 MFMA, through LDS.
//   W, U      fp16 MFMA against column-major xw / xu tiles in LDS, staged by an
//             exact identity-matrix MFMA transpose of each wave's rows.
// Precision: every MFMA operand of the state scan (W, b k 2^gk, qg, beta v, A, U,
// kg, Aqk) is fp16 with fp32 accumulation; gk, L, A are fp32.
// LDS stays under 80 KB at d = 128, so two workgroups share a CU; d = 256 takes
// 130 KB and one workgroup per CU.  From d = 128 on the workgroup has two
// channel groups of 4 waves (8 waves); d = 512 runs two channel passes.
#include <type_traits>

#include "gdn2_internal.h"

namespace memt {
namespace {

// Row-wise selection of 4 consecutive entries x[4 q + e] with q = lane group (0..3).
__device__ __forceinline__ f32x4 pick4(const float (&x)[16], int q) {
  f32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = q == 0 ? x[e] : q == 1 ? x[4 + e] : q == 2 ? x[8 + e] : x[12 + e];
  return r;
}

// Channel groups of 4 waves: the K channels (and V value columns) split into
// NCG groups, each handled by its own 4 waves; the L / Aqk tiles are summed
// over the groups through LDS.  At d = 128 two groups of 64 channels halve the
// registers per wave (at most 128: two 8-wave workgroups per CU, 16 waves to
// hide the load latency, against 8 with one group); d = 256 keeps 128 channels
// per group, one workgroup per CU (its LDS).
// (Four groups of 64 channels at d = 256, 16 waves in the one workgroup its LDS
// allows per CU, measured no faster than two groups.)
__host__ __device__ constexpr int wy_groups(int K) { return K >= 128 ? 2 : 1; }
// waves per SIMD the register budget is sized for
__host__ __device__ constexpr int wy_waves_per_simd(int K) { return K == 128 ? 4 : K < 128 ? 2 : 1; }
// Identity-matrix selectors: element j of lane (lr, lg) is 1 where the slot's channel
// (in the register order NAT names) is column lr of a 16-channel tile of parity
// `half`, so mfma(rows, sel) transposes
// a 16 x 16 tile exactly into the C layout (lane: 4 consecutive tokens of one channel).
template <bool NAT>
__device__ __forceinline__ void transpose_selectors(int lr, int lg, f16x8 (&sel)[2]) {
#pragma unroll
  for (int half = 0; half < 2; ++half)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool one = NAT ? 8 * lg + j == 16 * half + lr : (j >> 2) == half && 4 * lg + (j & 3) == lr;
      sel[half][j] = (_Float16)(one ? 1.f : 0.f);
    }
}

// Channel passes: d = 512 runs two passes of 256 channels through the same
// registers and LDS (wy_passes in gdn2_internal.h).

// RAW: the inputs are the memory block's projections (raw q, k, v, the decay
// projection, erase and write logits); the kernel forms g, beta, q_hat and
// k_til = sqrt_b * l2norm(k) itself, in the prologue's op order, and writes
// q_hat for the snapshot read.
template <int K, int V, bool CAUSAL, bool HAS_B, bool G_CUM, typename BetaT, bool RAW = false>
__global__ __launch_bounds__(256 * wy_groups(K), wy_waves_per_simd(K)) void wy_kernel(WyArgs a) {
  static_assert(!RAW || (!HAS_B && !G_CUM), "raw projections carry the erase gate in k and g un-summed");
  constexpr int C = kChunk;
  constexpr int KS = K / 32, VS = V / 32, VT = V / 16;  // whole-head counts (record layouts)
  constexpr int NCG = wy_groups(K), NT = 256 * NCG;
  // d > 256 runs the channels in NP passes of KP (VP) channels, each in the d = 256 layout
  constexpr int NP = wy_passes(K), KP = K / NP, VP = V / NP, KSP = KS / NP, VSP = VS / NP;
  constexpr int KSL = KSP / NCG, VSL = VSP / NCG, KTL = 2 * KSL, VTL = 2 * VSL;  // per channel group and pass
  static_assert(NP == 1 || (!CAUSAL && K == V), "d > 256: no causal output");
  constexpr int XP = C + 8;   // element pitch of the column-major xw / xu tiles
  constexpr int AP = C + 4;   // fp32 pitch of As_s
  constexpr int LQ = 16 + 4;  // fp32 pitch of a diagonal L tile
  constexpr int KBX = 6 * KSP * 64 * 8;  // fp16 elements of the six off-diagonal operands
  constexpr int XCH = KBX > KP * XP ? KBX : KP * XP;
  constexpr float kWide = 96.f;  // in-block decay span (log2) beyond which exact products are used

  // per-channel arrays hold one pass's KP channels
  __shared__ __attribute__((aligned(16))) float tot_s[4 * KP];    // block sums of g
  __shared__ __attribute__((aligned(16))) float first_s[4 * KP];  // g (or gk) of each block's first token
  __shared__ __attribute__((aligned(16))) float last_s[KP];       // gk of the last valid token (G_CUM)
  // per channel: rows 0-3 gk at the block starts, 4-6 2^(start_{w+1} - start_w),
  // 7-10 2^(gk_last - start_w), 11-14 2^start_w, 15 gk_last
  __shared__ __attribute__((aligned(16))) float fac_s[16 * KP];
  __shared__ __attribute__((aligned(16))) _Float16 xch_s[XCH];   // off-diagonal operands, then xw
  __shared__ __attribute__((aligned(16))) _Float16 xu_s[VP * XP];  // column-major beta v
  __shared__ __attribute__((aligned(16))) float As_s[C * AP];     // A, row-major
  __shared__ __attribute__((aligned(16))) float Ld_s[4 * 16 * LQ];
  _Float16* const xw_s = xch_s;
  __shared__ float nrm_s[RAW && NCG > 1 ? 2 * NCG * C : 1];  // per-group l2norm sums
  __shared__ float vmax_s[NT / 16];                           // max |beta v| per 16-lane row

  const int chunk = blockIdx.x, h = blockIdx.y, H = a.H;
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  constexpr bool NAT = K >= 256;  // natural channel order in registers (see the header)
  // first channel (within a channel step of 32) of the slots 4 half .. 4 half + 3
  auto quad = [&](int s, int half) { return NAT ? 32 * s + 8 * lg + 4 * half : 32 * s + 16 * half + 4 * lg; };
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);  // token block; uniform: scalar branches
  const int cg = __builtin_amdgcn_readfirstlane(tid >> 8);          // channel group
  const int cbl = cg * (KP / NCG), vcbl = cg * (VP / NCG);         // its first channel / value column in a pass
  const int sgl = cg * KSL, vgl = cg * VSL;                         // and its first channel / value step
  const int tok0 = a.chunk_tok0[chunk], len = a.chunk_len[chunk];
  const size_t unit = (size_t)chunk * H + h;
  const int t = 16 * wave + lr;
  const bool valid = t < len;
  const size_t rowK = ((size_t)(tok0 + (valid ? t : 0)) * H + h) * K;
  const size_t rowV = ((size_t)(tok0 + (valid ? t : 0)) * H + h) * V;

  using BetaRaw = typename std::conditional<sizeof(BetaT) == 4, f32x4, bf16x4>::type;
  // RAW: beta = bf16(sigmoid(write logit)), the reference's bf16 write gate
  auto beta_of = [](float x) { return RAW ? (float)(__bf16)sigmoid_bf16(x) : x; };
  f32x4 Lt[4], Qt[4];  // L and Aqk tiles (I = wave, J <= I), summed over the passes
  if constexpr (NP > 1) {
#pragma unroll
    for (int J = 0; J < 4; ++J) Lt[J] = Qt[J] = zero4();
  }
  f16x8 xw8[NP][KSL];  // xw rows of each pass, staged in LDS after the inverse
  // d > 256 from raw projections: the l2 norms of q and k span both passes, so
  // their sums come first (each pass reads its q and k again, from L2)
  float sq_tot = 0.f, sk_tot = 0.f;
  if constexpr (RAW && NP > 1) {
    const size_t tr = (size_t)(tok0 + (valid ? t : 0));
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int s = 0; s < KSL; ++s)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int c0 = h * K + p * KP + cbl + quad(s, half);
          const bf16x4 qq = *(const bf16x4*)(a.q + tr * a.q_stride + c0);
          const bf16x4 kk = *(const bf16x4*)(a.k + tr * a.k_stride + c0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sq_tot += (float)qq[e] * (float)qq[e];
            sk_tot += (float)kk[e] * (float)kk[e];
          }
        }
    sq_tot += __shfl_xor(sq_tot, 16, 64);
    sq_tot += __shfl_xor(sq_tot, 32, 64);
    sk_tot += __shfl_xor(sk_tot, 16, 64);
    sk_tot += __shfl_xor(sk_tot, 32, 64);
    if (lg == 0) {
      nrm_s[(cg * C + t) * 2] = sq_tot;
      nrm_s[(cg * C + t) * 2 + 1] = sk_tot;
    }
    lds_barrier();
    sq_tot = sk_tot = 0.f;
#pragma unroll
    for (int c2 = 0; c2 < NCG; ++c2) {
      sq_tot += nrm_s[(c2 * C + t) * 2];
      sk_tot += nrm_s[(c2 * C + t) * 2 + 1];
    }
  }
  // (at d = 512 the compiler declines the full unroll for size and keeps the
  // loop with xw8 in registers; forcing it measured slightly slower)
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int cb = p * KP + cbl, vcb = p * VP + vcbl;  // global channel / value column of this pass
    const int sg0 = p * KSP + sgl;                     // and global channel step
    // ---- loads: every per-token input of this lane's row, in slot order ----
    // Issued in the order of first use (g for the cumsum, then v and beta, then
    // k / b / q for the per-channel loop), so each phase waits only for its own
    // inputs and the cumsum and factor phases run while the rest is in flight.
    // Rows past the chunk end read row 0 of the chunk and are zeroed where used.
    constexpr bool WANT_Q = CAUSAL || RAW;
    bf16x8 kraw[KSL], braw[HAS_B ? KSL : 1], qraw[WANT_Q ? KSL : 1];
    float g[KSL][8];
    bf16x4 vraw[VSL][2];
    BetaRaw btraw[VSL][2];
    bf16x8 fraw[RAW ? KSL : 1], fbias[RAW ? KSL : 1], eraw[RAW ? KSL : 1];
    if constexpr (RAW) {
      // projection rows: q, k, decay and erase rows H*K wide, v and write rows H*V
      const size_t tr = (size_t)(tok0 + (valid ? t : 0));
#pragma unroll
      for (int s = 0; s < KSL; ++s)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int c0 = h * K + cb + quad(s, half);
          const bf16x4 ff = *(const bf16x4*)(a.f_raw + tr * a.f_stride + c0);
          const bf16x4 bb = *(const bf16x4*)(a.decay_bias + c0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            fraw[s][4 * half + e] = ff[e];
            fbias[s][4 * half + e] = bb[e];
          }
        }
      asm volatile("" ::: "memory");
      if constexpr (NP == 1) {  // d > 256 loads v and the write gate for the U product only
#pragma unroll
        for (int s = 0; s < VSL; ++s)
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int c0 = h * V + vcb + quad(s, half);
            vraw[s][half] = *(const bf16x4*)(a.v + tr * a.v_stride + c0);
            btraw[s][half] = *(const BetaRaw*)(a.w_raw + tr * a.w_stride + c0);
          }
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for (int s = 0; s < KSL; ++s)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int c0 = h * K + cb + quad(s, half);
          const bf16x4 kk = *(const bf16x4*)(a.k + tr * a.k_stride + c0);
          const bf16x4 ee = *(const bf16x4*)(a.e_raw + tr * a.e_stride + c0);
          const bf16x4 qq = *(const bf16x4*)(a.q + tr * a.q_stride + c0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            kraw[s][4 * half + e] = kk[e];
            eraw[s][4 * half + e] = ee[e];
            qraw[s][4 * half + e] = qq[e];
          }
        }
    } else {
#pragma unroll
    for (int s = 0; s < KSL; ++s)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const f32x4 gg = *(const f32x4*)(a.g + rowK + cb + quad(s, half));
#pragma unroll
        for (int e = 0; e < 4; ++e) g[s][4 * half + e] = gg[e];
      }
    asm volatile("" ::: "memory");
    if constexpr (NP == 1) {  // d > 256 loads v and beta for the U product only
#pragma unroll
      for (int s = 0; s < VSL; ++s) {
        if constexpr (NAT) {
          const int c0 = vcb + 32 * s + 8 * lg;
          const bf16x8 v8 = *(const bf16x8*)(a.v + rowV + c0);
          if constexpr (sizeof(BetaT) == 4) {
#pragma unroll
            for (int half = 0; half < 2; ++half)
              btraw[s][half] = *(const BetaRaw*)((const BetaT*)a.beta + rowV + c0 + 4 * half);
          } else {
            const bf16x8 b8 = *(const bf16x8*)((const BetaT*)a.beta + rowV + c0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              btraw[s][0][e] = b8[e];
              btraw[s][1][e] = b8[4 + e];
            }
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vraw[s][0][e] = v8[e];
            vraw[s][1][e] = v8[4 + e];
          }
        } else {
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int c0 = vcb + quad(s, half);
            vraw[s][half] = *(const bf16x4*)(a.v + rowV + c0);
            btraw[s][half] = *(const BetaRaw*)((const BetaT*)a.beta + rowV + c0);
          }
        }
      }
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int s = 0; s < KSL; ++s) {
      if constexpr (NAT) {
        const int c0 = cb + 32 * s + 8 * lg;
        kraw[s] = *(const bf16x8*)(a.k + rowK + c0);
        if constexpr (HAS_B) braw[s] = *(const bf16x8*)(a.b + rowK + c0);
        if constexpr (CAUSAL) qraw[s] = *(const bf16x8*)(a.q + rowK + c0);
      } else {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int c0 = cb + quad(s, half);
          const bf16x4 kk = *(const bf16x4*)(a.k + rowK + c0);
          bf16x4 bb{}, qq{};
          if constexpr (HAS_B) bb = *(const bf16x4*)(a.b + rowK + c0);
          if constexpr (CAUSAL) qq = *(const bf16x4*)(a.q + rowK + c0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            kraw[s][4 * half + e] = kk[e];
            if constexpr (HAS_B) braw[s][4 * half + e] = bb[e];
            if constexpr (CAUSAL) qraw[s][4 * half + e] = qq[e];
          }
        }
      }
    }
    }
    auto kf = [&](int s, int j) { return (float)kraw[s][j]; };
    auto bkf = [&](int s, int j) { return HAS_B ? (float)kraw[s][j] * (float)braw[s][j] : (float)kraw[s][j]; };
    auto qf = [&](int s, int j) { return CAUSAL ? (float)qraw[s][j] : 0.f; };

    // ---- cumsum: inclusive within the 16-token block, then block offsets ----
    const float neg_rate = RAW ? -gate_exp((float)a.decay_scale_log[h]) : 0.f;  // -exp(s_h), uniform
    float gk[KSL][8];
#pragma unroll
    for (int s = 0; s < KSL; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (RAW) {
          // g = -exp(s_h) * softplus(f + bias): natural-log decay, fp32
          g[s][j] = valid ? neg_rate * softplus_internal((float)fraw[s][j] + (float)fbias[s][j]) : 0.f;
        } else {
          g[s][j] = valid ? g[s][j] : 0.f;
        }
        gk[s][j] = G_CUM ? g[s][j] : row_inclusive_scan(g[s][j]);
      }
#pragma unroll
    for (int s = 0; s < KSL; ++s)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int c0 = cbl + quad(s, half);
        const f32x4 gkv{gk[s][4 * half], gk[s][4 * half + 1], gk[s][4 * half + 2], gk[s][4 * half + 3]};
        const f32x4 gv{g[s][4 * half], g[s][4 * half + 1], g[s][4 * half + 2], g[s][4 * half + 3]};
        if (!G_CUM && lr == 15) *(f32x4*)(&tot_s[wave * KP + c0]) = gkv;
        if (lr == 0) *(f32x4*)(&first_s[wave * KP + c0]) = gv;
        if (G_CUM && t == len - 1) *(f32x4*)(&last_s[c0]) = gv;
      }
    lds_barrier();
#pragma unroll
    for (int s = 0; s < KSL; ++s)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int c0 = cbl + quad(s, half);
        if constexpr (!G_CUM) {
          f32x4 base = zero4();
          for (int w2 = 0; w2 < wave; ++w2) base += *(const f32x4*)(&tot_s[w2 * KP + c0]);
#pragma unroll
          for (int e = 0; e < 4; ++e) gk[s][4 * half + e] = (base[e] + gk[s][4 * half + e]) * kRcpLn2;
        } else if (!valid) {
          const f32x4 lv = *(const f32x4*)(&last_s[c0]);
#pragma unroll
          for (int e = 0; e < 4; ++e) gk[s][4 * half + e] = lv[e];
        }
      }
    for (int idx = tid; idx < 2 * KP; idx += NT) {
      // two threads per channel: part 0 writes the block starts, their ratios and gk_last,
      // part 1 the powers used by kg and by xw / qg
      const int c = idx % KP, part = idx / KP;
      float ref[4], last;
      if constexpr (!G_CUM) {
        // same summation order as the per-lane offsets above, so fa == 1 exactly at block starts
        float run = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
          ref[w2] = (run + first_s[w2 * KP + c]) * kRcpLn2;
          run += tot_s[w2 * KP + c];
        }
        last = run * kRcpLn2;
      } else {
        last = last_s[c];
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) ref[w2] = (16 * w2 < len) ? first_s[w2 * KP + c] : last;
      }
      if (part == 0) {
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
          fac_s[w2 * KP + c] = ref[w2];
          if (w2 < 3) fac_s[(4 + w2) * KP + c] = fast_exp2(ref[w2 + 1] - ref[w2]);
        }
        fac_s[15 * KP + c] = last;
        a.out.decay[unit * K + p * KP + c] = fast_exp2(last);
      } else {
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
          fac_s[(7 + w2) * KP + c] = fast_exp2(last - ref[w2]);
          fac_s[(11 + w2) * KP + c] = fast_exp2(ref[w2]);
        }
      }
    }
    if constexpr (NP == 1) {
      // the unit's max |beta v| (rows past the chunk end repeat row 0), for the
      // value exponent of U; d > 256 forms it per pass in stage_x
      float vmax = 0.f;
#pragma unroll
      for (int s = 0; s < VSL; ++s)
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            vmax = fmaxf(vmax, fabsf((float)vraw[s][half][e] * beta_of((float)btraw[s][half][e])));
      vmax = row_max_nonneg(vmax);  // DPP row maxima: one partial per 16 lanes
      if (lr == 15) vmax_s[(tid >> 6) * 4 + lg] = vmax;
    }
    lds_barrier();

    float uscale = 1.f;  // 2^-uexp
    if constexpr (NP == 1) {
      float m = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < NT / 16; ++w2) m = fmaxf(m, vmax_s[w2]);
      const int uexp = value_exponent(m);
      uscale = ldexpf(1.f, -uexp);
      if (tid == 0) a.out.uexp[unit] = uexp;
    }
    f16x8 sel_h[2];
    transpose_selectors<NAT>(lr, lg, sel_h);
    // beta v * 2^-uexp to LDS, column-major (channel rows, token columns); read by the U product
#pragma unroll
    for (int s = 0; s < (NP == 1 ? VSL : 0); ++s) {
      f16x8 xu8;
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
          const float bt = beta_of((float)btraw[s][half][e]);
          xu8[4 * half + e] = (_Float16)(valid ? (float)vraw[s][half][e] * bt * uscale : 0.f);
        }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ct = 2 * (vgl + s) + half;
        const f32x4 tr = mfma_f16(xu8, sel_h[half], zero4());
        f16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (_Float16)tr[e];
        *(f16x4*)(&xu_s[(16 * ct + lr) * XP + 16 * wave + 4 * lg]) = o4;
      }
    }
    if constexpr (RAW) {
      // q_hat = bf16(q / sqrt(sum q^2 + eps)), k_til = bf16(sqrt_b * bf16(k / sqrt(sum k^2 + eps)))
      // with sqrt_b = bf16(exp(logsigmoid(e) / 2)); a token's channels sit on the four lanes lr + 16 i
      float sq = sq_tot, sk = sk_tot;  // d > 256: both passes' sums, from before the loop
      if constexpr (NP == 1) {
#pragma unroll
        for (int s = 0; s < KSL; ++s)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float qv = (float)qraw[s][j], kv = (float)kraw[s][j];
            sq += qv * qv;
            sk += kv * kv;
          }
        sq += __shfl_xor(sq, 16, 64);
        sq += __shfl_xor(sq, 32, 64);
        sk += __shfl_xor(sk, 16, 64);
        sk += __shfl_xor(sk, 32, 64);
      }
      if constexpr (NCG > 1 && NP == 1) {
        // each group holds K / NCG of the token's channels
        if (lg == 0) {
          nrm_s[(cg * C + t) * 2] = sq;
          nrm_s[(cg * C + t) * 2 + 1] = sk;
        }
        lds_barrier();
        sq = sk = 0.f;
#pragma unroll
        for (int c2 = 0; c2 < NCG; ++c2) {
          sq += nrm_s[(c2 * C + t) * 2];
          sk += nrm_s[(c2 * C + t) * 2 + 1];
        }
      }
      const float rq = 1.f / sqrtf(sq + a.eps), rk = 1.f / sqrtf(sk + a.eps);
#pragma unroll
      for (int s = 0; s < KSL; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float sbv = (float)(__bf16)sqrt_sigmoid_bf16((float)eraw[s][j]);
          const float khat = (float)(__bf16)((float)kraw[s][j] * rk);
          kraw[s][j] = (__bf16)(sbv * khat);
          qraw[s][j] = (__bf16)((float)qraw[s][j] * rq);
        }
      if (valid && a.q_hat != nullptr) {
        __bf16* qo = a.q_hat + ((size_t)(tok0 + t) * H + h) * K;
#pragma unroll
        for (int s = 0; s < KSL; ++s)
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            bf16x4 o4;
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = qraw[s][4 * half + e];
            *(bf16x4*)(qo + cb + quad(s, half)) = o4;
          }
      }
    }
    if (!valid) {
#pragma unroll
      for (int s = 0; s < KSL; ++s) {
        kraw[s] = bf16x8{};
        if constexpr (HAS_B) braw[s] = bf16x8{};
        if constexpr (WANT_Q) qraw[s] = bf16x8{};
      }
    }

    // ---- in-block decay span: a wide block takes exact diagonal products ----
    float span = 0.f;
#pragma unroll
    for (int s = 0; s < KSL; ++s)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const f32x4 r4 = *(const f32x4*)(&fac_s[wave * KP + cbl + quad(s, half)]);
#pragma unroll
        for (int e = 0; e < 4; ++e) span = fmaxf(span, r4[e] - gk[s][4 * half + e]);
      }
    const bool wide = __builtin_amdgcn_readfirstlane(wave_max(span) > kWide ? 1 : 0) != 0;
    f32x4 Ld4 = zero4(), Qd4 = zero4();  // diagonal L / Aqk tiles (row lr, cols 4 lg + e)
    if (wide) {
      // lane (lr, lg) sums its own channels for the columns j of the block, reading the
      // column tokens through shuffles inside its lane group; the four groups then add up
      float pl[16], pq[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) pl[j] = pq[j] = 0.f;
#pragma unroll
      for (int s = 0; s < KSL; ++s)
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const float gj = __shfl(gk[s][jj], j + 16 * lg, 64);
            const float kj = __shfl(kf(s, jj), j + 16 * lg, 64);
            const float f = j <= lr ? fast_exp2(gk[s][jj] - gj) : 0.f;
            pl[j] += bkf(s, jj) * kj * f;
            if constexpr (CAUSAL) pq[j] += qf(s, jj) * kj * f;
          }
        }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        pl[j] += __shfl_xor(pl[j], 16, 64);
        pl[j] += __shfl_xor(pl[j], 32, 64);
        if constexpr (CAUSAL) {
          pq[j] += __shfl_xor(pq[j], 16, 64);
          pq[j] += __shfl_xor(pq[j], 32, 64);
        }
      }
      Ld4 = pick4(pl, lg);
      Qd4 = pick4(pq, lg);
    }

    // ---- per channel step: factors, operands, the diagonal tiles and the outputs ----
    // Off-diagonal column operands are built by wave J for row blocks I > J:
    // k 2^(start_I - gk) = k (1/fa) prod_{w=J}^{I-1} 2^(start_{w+1} - start_w), each factor <= 1.
    auto pair_index = [](int I, int J) { return J * (7 - J) / 2 + (I - J - 1); };
    f16x8 a16[KSL], aq16[CAUSAL ? KSL : 1];
    _Float16* const kg_out = a.out.kgT + unit * (size_t)(C * K);
#pragma unroll
    for (int s = 0; s < KSL; ++s) {
      f16x8 qg8, kg8;
      float avs[8], kbs[8], qvs[8];
      float base[8];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int c0 = cbl + quad(s, half);
        const f32x4 r4 = *(const f32x4*)(&fac_s[wave * KP + c0]);
        const f32x4 gw = *(const f32x4*)(&fac_s[(7 + wave) * KP + c0]);
        const f32x4 ew = *(const f32x4*)(&fac_s[(11 + wave) * KP + c0]);
        const int wn = wave < 3 ? wave : 2;
        const f32x4 dj = *(const f32x4*)(&fac_s[(4 + wn) * KP + c0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * half + e;
          const float d = gk[s][j] - r4[e];  // <= 0
          const float fa = fast_exp2(d), ifa = fast_exp2(-d);
          const float av = bkf(s, j) * fa;
          avs[j] = av;
          a16[s][j] = (_Float16)av;
          xw8[p][s][j] = (_Float16)(av * ew[e]);
          const float kbv = kf(s, j) * ifa;
          kbs[j] = kbv;
          kg8[j] = (_Float16)(kbv * gw[e]);
          base[j] = kbv * dj[e];
          if constexpr (CAUSAL) {
            const float qv = qf(s, j) * fa;
            qvs[j] = qv;
            aq16[s][j] = (_Float16)qv;
            qg8[j] = (_Float16)(qv * ew[e]);
          }
        }
      }
      if (wide) {
        // exact factors where the re-centred ones could overflow (a scalar branch,
        // so their exp2s run only for such blocks)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int c0 = cbl + quad(s, half);
          const f32x4 lastv = *(const f32x4*)(&fac_s[15 * KP + c0]);
          const int wn = wave < 3 ? wave : 2;
          const f32x4 rn = *(const f32x4*)(&fac_s[(wn + 1) * KP + c0]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = 4 * half + e;
            kg8[j] = (_Float16)(kf(s, j) * fast_exp2(lastv[e] - gk[s][j]));
            base[j] = kf(s, j) * fast_exp2(rn[e] - gk[s][j]);
          }
        }
      }
      if (!wide) {
        // fp32 MFMA, one channel per lane group and step: exact products, full range
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          Ld4 = mfma_f32(kbs[j], avs[j], Ld4);
          if constexpr (CAUSAL) Qd4 = mfma_f32(kbs[j], qvs[j], Qd4);
        }
      }
      if constexpr (CAUSAL) {
        f16x8 qp = qg8;
        if constexpr (NAT) {
          // to the scan's channel order through this wave's 1280 bytes of As_s (free
          // until the inverse): row lr holds the 32 channels of the step at a
          // 40-element pitch; LDS operations of one wave complete in order
          _Float16* const qs = (_Float16*)As_s + (tid >> 6) * 640 + lr * 40;
          *(f16x8*)(qs + 8 * lg) = qg8;
          __builtin_amdgcn_wave_barrier();
          asm volatile("" ::: "memory");
          const f16x4 lo = *(const f16x4*)(qs + 4 * lg), hi = *(const f16x4*)(qs + 16 + 4 * lg);
          asm volatile("" ::: "memory");
          __builtin_amdgcn_wave_barrier();
          qp = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        *(f16x8*)(a.out.qg + unit * (size_t)(C * K) + ((size_t)(wave * KS + sg0 + s) * 64 + lane) * 8) = qp;
      }
      // kg^T to global as P-frags (rows = channels, reduction = tokens)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ct = 2 * (sg0 + s) + half;
        const f32x4 tr = mfma_f16(kg8, sel_h[half], zero4());
        f16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (_Float16)tr[e];
        *(f16x4*)(kg_out + ((size_t)(ct * 2 + (wave >> 1)) * 64 + lane) * 8 + (wave & 1) * 4) = o4;
      }
      if (wave < 3) {
#pragma unroll
        for (int I = 1; I < 4; ++I) {
          if (I <= wave) continue;
          if (I > wave + 1) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
              const f32x4 dn = *(const f32x4*)(&fac_s[(4 + I - 1) * KP + cbl + quad(s, half)]);
#pragma unroll
              for (int e = 0; e < 4; ++e) base[4 * half + e] *= dn[e];
            }
          }
          f16x8 op;
#pragma unroll
          for (int j = 0; j < 8; ++j) op[j] = (_Float16)base[j];
          *(f16x8*)(&xch_s[((size_t)(pair_index(I, wave) * KSP + sgl + s) * 64 + lane) * 8]) = op;
        }
      }
    }
    lds_barrier();  // off-diagonal operands visible

    // ---- this pass's share of the L and Aqk tiles, transposed: lane holds row lr, cols 4 lg + e ----
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      if constexpr (NP == 1) {
        Lt[J] = J == wave ? Ld4 : zero4();
        Qt[J] = J == wave ? Qd4 : zero4();
      } else if (J == wave) {
        Lt[J] += Ld4;
        Qt[J] += Qd4;
      }
    }
#pragma unroll
    for (int J = 0; J < 3; ++J) {
      if (J >= wave) continue;
#pragma unroll
      for (int s = 0; s < KSL; ++s) {
        const f16x8 op = *(const f16x8*)(&xch_s[((size_t)(pair_index(wave, J) * KSP + sgl + s) * 64 + lane) * 8]);
        Lt[J] = mfma_f16(op, a16[s], Lt[J]);
        if constexpr (CAUSAL) Qt[J] = mfma_f16(op, aq16[s], Qt[J]);
      }
    }
  }  // pass
  if constexpr (NCG > 1) {
    // sum the groups' partial tiles into group 0 (tiles J <= wave: 10 per group
    // and matrix), through the off-diagonal operand buffer, dead once read; FIT
    // groups' tiles fit it at once, so more groups take several rounds
    constexpr int PER_GROUP = 2 * 10 * 64 * 4;                // floats of one group's L and Aqk tiles
    constexpr int FIT = (int)(XCH * sizeof(_Float16) / sizeof(float)) / PER_GROUP;
    static_assert(FIT >= 1, "reduction buffer");
    float* red = (float*)xch_s;
    auto slot = [&](int idx, int q2, int J) { return (((idx * 2 + q2) * 10 + wave * (wave + 1) / 2 + J) * 64 + lane) * 4; };
#pragma unroll
    for (int r0 = 1; r0 < NCG; r0 += FIT) {
      lds_barrier();  // every wave is done with the buffer's previous contents
      if (cg >= r0 && cg < r0 + FIT) {
#pragma unroll
        for (int J = 0; J < 4; ++J) {
          if (J > wave) continue;
          *(f32x4*)(&red[slot(cg - r0, 0, J)]) = Lt[J];
          if constexpr (CAUSAL) *(f32x4*)(&red[slot(cg - r0, 1, J)]) = Qt[J];
        }
      }
      lds_barrier();
      if (cg == 0) {
#pragma unroll
        for (int i = 0; i < FIT; ++i) {
          if (r0 + i >= NCG) continue;
#pragma unroll
          for (int J = 0; J < 4; ++J) {
            if (J > wave) continue;
            Lt[J] += *(const f32x4*)(&red[slot(i, 0, J)]);
            if constexpr (CAUSAL) Qt[J] += *(const f32x4*)(&red[slot(i, 1, J)]);
          }
        }
      }
    }
  }
  // masks, the Aqk record, the inverse: group 0 (the other groups wait at the barriers)
  f32x4 Aii = zero4();
  if (cg == 0) {
  // masks: L strictly lower, Aqk lower with the diagonal, scaled
#pragma unroll
  for (int J = 0; J < 4; ++J) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int col = 4 * lg + e;
      const bool diag = J == wave;
      if (J > wave || (diag && col >= lr)) Lt[J][e] = 0.f;
      if constexpr (CAUSAL) Qt[J][e] = (J > wave || (diag && col > lr)) ? 0.f : a.scale * Qt[J][e];
    }
  }
  if constexpr (CAUSAL) {
    _Float16* aq_out = a.out.Aqk + unit * (size_t)(C * C);
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      f16x4 o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = (_Float16)Qt[J][e];
      *(f16x4*)(aq_out + ((size_t)(wave * 2 + (J >> 1)) * 64 + lane) * 8 + (J & 1) * 4) = o4;
    }
  }

  // ---- A_II by row substitution: x (I + L_II) = e_lr, x[m] = d_lm - sum_{p>m} x[p] L[p][m] ----
  {
    float* Ld = Ld_s + wave * 16 * LQ;
    f32x4 ld4 = zero4();
#pragma unroll
    for (int J = 0; J < 4; ++J)
      if (J == wave) ld4 = Lt[J];
    *(f32x4*)(&Ld[lr * LQ + 4 * lg]) = ld4;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's own tile is in LDS
    __builtin_amdgcn_wave_barrier();
    float x[16], acc[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) acc[m] = 0.f;
#pragma unroll
    for (int p = 15; p >= 0; --p) {
      x[p] = (p == lr ? 1.f : 0.f) - acc[p];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        if (4 * q4 >= p) continue;
        const f32x4 row = *(const f32x4*)(&Ld[p * LQ + 4 * q4]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * q4 + e < p) acc[4 * q4 + e] += x[p] * row[e];
      }
    }
    Aii = pick4(x, lg);
  }
  *(f32x4*)(&As_s[(16 * wave + lr) * AP + 16 * wave + 4 * lg]) = Aii;
#pragma unroll
  for (int J = 0; J < 4; ++J)
    if (J > wave) *(f32x4*)(&As_s[(16 * wave + lr) * AP + 16 * J + 4 * lg]) = zero4();
  }
  lds_barrier();  // A_II visible; the off-diagonal operands are dead

  // xw (and, d > 256, beta v, loaded here) of pass p, column-major (channel rows,
  // token columns), by identity transposes into this group's tiles of the pass
  auto stage_x = [&](int p) {
    f16x8 sel[2];
    transpose_selectors<NAT>(lr, lg, sel);
#pragma unroll
    for (int ct = 0; ct < KTL; ++ct) {
      const f32x4 tr = mfma_f16(xw8[p][ct >> 1], sel[ct & 1], zero4());
      f16x4 o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = (_Float16)tr[e];
      *(f16x4*)(&xw_s[(16 * (2 * sgl + ct) + lr) * XP + 16 * wave + 4 * lg]) = o4;
    }
    if constexpr (NP > 1) {
      const int vcb = p * VP + vcbl;
      const size_t tr = (size_t)(tok0 + (valid ? t : 0));
      auto load_vb = [&](int s, int half, bf16x4& v4, BetaRaw& b4) {
        const int c0 = vcb + quad(s, half);
        if constexpr (RAW) {  // projection rows; beta = bf16(sigmoid(write logit))
          v4 = *(const bf16x4*)(a.v + tr * a.v_stride + h * V + c0);
          b4 = *(const BetaRaw*)(a.w_raw + tr * a.w_stride + h * V + c0);
        } else {
          v4 = *(const bf16x4*)(a.v + rowV + c0);
          b4 = *(const BetaRaw*)((const BetaT*)a.beta + rowV + c0);
        }
      };
      // this pass's beta v in registers, its max |beta v| (DPP row maxima, one
      // partial per 16 lanes through LDS) and then its value exponent
      float pv[VSL][8];
      float vmax = 0.f;
#pragma unroll
      for (int s = 0; s < VSL; ++s)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          bf16x4 v4;
          BetaRaw b4;
          load_vb(s, half, v4, b4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pv[s][4 * half + e] = valid ? (float)v4[e] * beta_of((float)b4[e]) : 0.f;
            vmax = fmaxf(vmax, fabsf(pv[s][4 * half + e]));
          }
        }
      vmax = row_max_nonneg(vmax);
      if (lr == 15) vmax_s[(tid >> 6) * 4 + lg] = vmax;
      lds_barrier();
      float m = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < NT / 16; ++w2) m = fmaxf(m, vmax_s[w2]);
      const int uexp = value_exponent(m);
      const float us = ldexpf(1.f, -uexp);
      if (tid == 0) a.out.uexp[unit * NP + p] = uexp;
#pragma unroll
      for (int s = 0; s < VSL; ++s) {
        f16x8 xu8;
#pragma unroll
        for (int j = 0; j < 8; ++j) xu8[j] = (_Float16)(pv[s][j] * us);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int ct = 2 * (vgl + s) + half;
          const f32x4 tr = mfma_f16(xu8, sel[half], zero4());
          f16x4 o4;
#pragma unroll
          for (int e = 0; e < 4; ++e) o4[e] = (_Float16)tr[e];
          *(f16x4*)(&xu_s[(16 * ct + lr) * XP + 16 * wave + 4 * lg]) = o4;
        }
      }
    }
  };
  if constexpr (NP == 1) stage_x(0);

  // ---- A_IJ = -A_II sum_{M=J}^{I-1} L_IM A_MJ, stage d = I - J ----
#pragma unroll
  for (int d = 1; d <= 3; ++d) {
    if (cg == 0 && wave >= d) {
      const int J = wave - d;
      f32x4 T = zero4();
#pragma unroll
      for (int M = 0; M < 3; ++M) {
        if (M < J || M >= wave) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float bv = As_s[(16 * M + 4 * lg + e) * AP + 16 * J + lr];
          T = mfma_f32(Lt[M][e], bv, T);
        }
      }
      f32x4 R = zero4();
#pragma unroll
      for (int e = 0; e < 4; ++e) R = mfma_f32(Aii[e], T[e], R);
#pragma unroll
      for (int e = 0; e < 4; ++e) As_s[(16 * wave + 4 * lg + e) * AP + 16 * J + lr] = -R[e];
    }
    lds_barrier();
  }

  // ---- W^T = xw^T A^T and U = A xu (fp16), row block R = wave ----
  {
    const int R = wave;
    constexpr int NS = 2;  // 32-token reduction steps
    f16x8 ah[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const f32x4 r4 = *(const f32x4*)(&As_s[(16 * R + lr) * AP + 32 * s + 16 * half + 4 * lg]);
#pragma unroll
        for (int e = 0; e < 4; ++e) ah[s][4 * half + e] = (_Float16)r4[e];
      }
    }
    const bool two = R >= 2;  // row blocks 0, 1 have no entries past token 31
    _Float16* W_out = a.out.W + unit * (size_t)(C * K);
    _Float16* U_out = a.out.U + unit * (size_t)(C * V);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if constexpr (NP > 1) {
        if (p > 0) lds_barrier();  // the previous pass's tiles are consumed
        stage_x(p);
        lds_barrier();
      }
#pragma unroll
      for (int ctl = 0; ctl < KTL; ++ctl) {
        const int ct = 2 * sgl + ctl, ctg = 2 * (p * KSP + sgl) + ctl;  // tile in LDS / in the record
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          if (s == 1 && !two) continue;
          const _Float16* col = xw_s + (16 * ct + lr) * XP + 32 * s + 4 * lg;
          const f16x4 lo = *(const f16x4*)col;
          const f16x4 hi = *(const f16x4*)(col + 16);
          const f16x8 xa{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          acc = mfma_f16(xa, ah[s], acc);
        }
        f16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (_Float16)acc[e];
        *(f16x4*)(W_out + ((size_t)(R * KS + (ctg >> 1)) * 64 + lane) * 8 + (ctg & 1) * 4) = o4;
      }
#pragma unroll
      for (int ctl = 0; ctl < VTL; ++ctl) {
        const int ct = 2 * vgl + ctl, ctg = 2 * (p * VSP + vgl) + ctl;
        f32x4 acc = zero4();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          if (s == 1 && !two) continue;
          const _Float16* col = xu_s + (16 * ct + lr) * XP + 32 * s + 4 * lg;
          const f16x4 lo = *(const f16x4*)col;
          const f16x4 hi = *(const f16x4*)(col + 16);
          const f16x8 xb{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          acc = mfma_f16(ah[s], xb, acc);
        }
        f16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (_Float16)acc[e];
        *(f16x4*)(U_out + ((size_t)(R * VT + ctg) * 64 + lane) * 4) = o4;
      }
    }  // pass
  }
  if (a.A_ref != nullptr) {
    for (int idx = tid; idx < len * C; idx += NT) {
      const int tt = idx / C, j = idx % C;
      a.A_ref[((size_t)(tok0 + tt) * H + h) * C + j] = (__bf16)As_s[tt * AP + j];
    }
  }
}

template <int K, int V, bool CAUSAL>
hipError_t launch_raw(const WyArgs& a, int n_chunk, hipStream_t stream) {
  hipLaunchKernelGGL((wy_kernel<K, V, CAUSAL, false, false, __bf16, true>), dim3(n_chunk, a.H),
                     dim3(256 * wy_groups(K)), 0, stream, a);
  return hipGetLastError();
}

template <int K, int V, bool CAUSAL, bool HAS_B, bool G_CUM>
hipError_t launch_t(const WyArgs& a, int n_chunk, bool beta_bf16, hipStream_t stream) {
  dim3 grid(n_chunk, a.H), block(256 * wy_groups(K));
  if (beta_bf16)
    hipLaunchKernelGGL((wy_kernel<K, V, CAUSAL, HAS_B, G_CUM, __bf16>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((wy_kernel<K, V, CAUSAL, HAS_B, G_CUM, float>), grid, block, 0, stream, a);
  return hipGetLastError();
}

template <int K, int V>
hipError_t launch_kv(const WyArgs& a, int n_chunk, bool causal, bool g_cum, bool beta_bf16,
                     hipStream_t stream) {
  const bool has_b = a.b != nullptr;
  if constexpr (wy_passes(K) > 1) {
    // d > 256: the final-state and snapshot-read modes only
    if (causal) return hipErrorInvalidValue;
    if (a.f_raw != nullptr) return launch_raw<K, V, false>(a, n_chunk, stream);
    if (g_cum) return has_b ? launch_t<K, V, false, true, true>(a, n_chunk, beta_bf16, stream)
                            : launch_t<K, V, false, false, true>(a, n_chunk, beta_bf16, stream);
    return has_b ? launch_t<K, V, false, true, false>(a, n_chunk, beta_bf16, stream)
                 : launch_t<K, V, false, false, false>(a, n_chunk, beta_bf16, stream);
  } else {
    if (a.f_raw != nullptr)
      return causal ? launch_raw<K, V, true>(a, n_chunk, stream) : launch_raw<K, V, false>(a, n_chunk, stream);
#define MEMT_WY_CASE(CA, HB, GC) \
    if (causal == CA && has_b == HB && g_cum == GC) return launch_t<K, V, CA, HB, GC>(a, n_chunk, beta_bf16, stream);
    MEMT_WY_CASE(false, false, false)
    MEMT_WY_CASE(false, true, false)
    MEMT_WY_CASE(true, false, false)
    MEMT_WY_CASE(true, true, false)
    MEMT_WY_CASE(false, false, true)
    MEMT_WY_CASE(false, true, true)
    MEMT_WY_CASE(true, false, true)
    MEMT_WY_CASE(true, true, true)
#undef MEMT_WY_CASE
    return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_wy(const WyArgs& a, int n_chunk, int K, int V, bool causal, bool g_cumulative,
                     bool beta_bf16, hipStream_t stream) {
  if (n_chunk == 0) return hipSuccess;
  if (K == 64 && V == 64) return launch_kv<64, 64>(a, n_chunk, causal, g_cumulative, beta_bf16, stream);
  if (K == 128 && V == 128) return launch_kv<128, 128>(a, n_chunk, causal, g_cumulative, beta_bf16, stream);
  if (K == 256 && V == 256) return launch_kv<256, 256>(a, n_chunk, causal, g_cumulative, beta_bf16, stream);
  if (K == 512 && V == 512) return launch_kv<512, 512>(a, n_chunk, causal, g_cumulative, beta_bf16, stream);
  return hipErrorInvalidValue;
}

}  // namespace memt
