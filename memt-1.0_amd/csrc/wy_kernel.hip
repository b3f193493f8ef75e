// WY stage of the chunked GDN-2 update, one workgroup per (chunk, head).
//
// For a chunk of C <= 64 tokens (rows past the chunk end are zero padded):
//   gk    = 1/ln2 * cumsum_chunk(g)                       (FLA/ops/utils/cumsum.py:116-133)
//   L     = strictly lower, L[i,j] = sum_c (b k)_ic k_jc 2^(gk_ic - gk_jc)
//                                                          (FLA/ops/gdn2/chunk_intra_token_parallel.py:111-123,
//                                                           FLA/ops/gdn2/chunk_intra.py:233-299)
//   A     = (I + L)^-1                                     (chunk_intra.py:326-395)
//   W     = A (b k 2^gk),  U = A (beta v)                  (FLA/ops/gdn2/wy_fast.py:92-142)
// Outputs go to the workspace as MFMA operand fragments of the state scan
// (P-frags for W, qg, kg^T and Aqk; a C-frag for U).
//   kg    = k 2^(gk_last - gk), decay = 2^gk_last          (wy_fast.py:125-139)
//   Aqk   = scale * sum_c q_ic k_jc 2^(gk_ic - gk_jc), j <= i, qg = q 2^gk   (causal output only)
//
// Precision: the erase path (W, b k 2^gk) is bf16; the value path (beta v, A, U,
// kg, Aqk) is fp16 with fp32 accumulation; gk, L, A are fp32.  The diagonal
// 16x16 blocks of L use fp32 MFMA with factors re-centred at the block start;
// a block whose in-block decay exceeds 2^64 takes an exact pairwise path.
// Off-diagonal blocks are re-centred at the row block start, so both operand
// factors are <= 1 and fp16 MFMA is safe.  The inverse is formed block-wise:
// forward substitution on the diagonal blocks, then
// A_IJ = -A_II sum_{J<=M<I} L_IM A_MJ with fp32 MFMA.
#include "gdn2_internal.h"

namespace memt {
namespace {

template <int K, int V, bool CAUSAL, bool HAS_B, bool G_CUM, typename BetaT>
__global__ __launch_bounds__(256) void wy_kernel(WyArgs a) {
  constexpr int C = kChunk;
  constexpr int KP = K + 4;   // fp32 row pitch of gk_s
  constexpr int KB = K + 8;   // bf16 row pitch of k_s / q_s / b_s / W staging
  constexpr int CB = C + 8;   // row pitch of the column-major xw_s / xu_s
  constexpr int LP = C + 4;   // fp32 row pitch of L_s / A_s / Aqk_s
  constexpr int GKS = (C * KP * 4 > V * CB * 2 ? C * KP * 4 : V * CB * 2) / 4;
  static_assert(C * KB * 2 <= K * CB * 2 + 1024, "W staging must fit in xw_s");

  __shared__ __attribute__((aligned(16))) float gk_s[GKS];  // later: xu_s (f16 [V][CB])
  __shared__ __attribute__((aligned(16))) __bf16 k_s[C * KB];
  __shared__ __attribute__((aligned(16))) __bf16 q_s[CAUSAL ? C * KB : 8];
  __shared__ __attribute__((aligned(16))) __bf16 b_s[HAS_B ? C * KB : 8];
  __shared__ __attribute__((aligned(16))) __bf16 xw_s[K * CB + 512];  // later: W staging [C][KB]
  __shared__ __attribute__((aligned(16))) float L_s[C * LP];
  __shared__ __attribute__((aligned(16))) float A_s[C * LP];
  __shared__ __attribute__((aligned(16))) float Aqk_s[CAUSAL ? C * LP : 4];
  __shared__ float tot_s[4 * K];

  const int chunk = blockIdx.x, h = blockIdx.y, H = a.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int tok0 = a.chunk_tok0[chunk];
  const int len = a.chunk_len[chunk];
  const size_t unit = (size_t)chunk * H + h;

  // ---- phase 1: issue every global load of the chunk at once (k, q, b, g and
  //      the v / beta operands of phase 4), stage k / q / b, decay cumsum ----
  constexpr int K8 = K / 8;
  constexpr int V8 = V / 8;
  constexpr int NKL = C * K8 / 256;  // 16-byte k/q/b loads per thread
  constexpr int NVL = C * V8 / 256;  // 8-element v/beta groups per thread
  static_assert(NKL * 256 == C * K8 && NVL * 256 == C * V8, "load tiling");
  constexpr int TPC = (256 / K) < 1 ? 1 : (256 / K);  // threads per channel
  constexpr int SEG = C / TPC;
  u32x4 kv[NKL], qv[CAUSAL ? NKL : 1], bv[HAS_B ? NKL : 1];
#pragma unroll
  for (int i = 0; i < NKL; ++i) {
    const int idx = tid + 256 * i;
    const int t = idx / K8, c8 = (idx % K8) * 8;
    const size_t goff = ((size_t)(tok0 + t) * H + h) * K + c8;
    kv[i] = u32x4{0u, 0u, 0u, 0u};
    if constexpr (CAUSAL) qv[i] = u32x4{0u, 0u, 0u, 0u};
    if constexpr (HAS_B) bv[i] = u32x4{0u, 0u, 0u, 0u};
    if (t < len) {
      kv[i] = *(const u32x4*)(a.k + goff);
      if constexpr (CAUSAL) qv[i] = *(const u32x4*)(a.q + goff);
      if constexpr (HAS_B) bv[i] = *(const u32x4*)(a.b + goff);
    }
  }
  float gv[SEG];
  {
    const int c = tid % K, seg = tid / K;
#pragma unroll
    for (int i = 0; i < SEG; ++i) {
      const int t = seg * SEG + i;
      gv[i] = (tid < K * TPC && t < len) ? a.g[((size_t)(tok0 + t) * H + h) * K + c] : 0.f;
    }
  }
  bf16x8 vreg[NVL];
  float breg[NVL][8];
#pragma unroll
  for (int i = 0; i < NVL; ++i) {
    const int idx = tid + 256 * i;
    const int t = idx / V8, c8 = (idx % V8) * 8;
    const size_t goff = ((size_t)(tok0 + t) * H + h) * V + c8;
    if (t < len) {
      vreg[i] = *(const bf16x8*)(a.v + goff);
      if constexpr (sizeof(BetaT) == 4) {
        const f32x4 b0 = *(const f32x4*)((const float*)a.beta + goff);
        const f32x4 b1 = *(const f32x4*)((const float*)a.beta + goff + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          breg[i][e] = b0[e];
          breg[i][4 + e] = b1[e];
        }
      } else {
        const bf16x8 bb = *(const bf16x8*)((const __bf16*)a.beta + goff);
#pragma unroll
        for (int e = 0; e < 8; ++e) breg[i][e] = (float)bb[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vreg[i][e] = (__bf16)0.f;
        breg[i][e] = 0.f;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NKL; ++i) {
    const int idx = tid + 256 * i;
    const int t = idx / K8, c8 = (idx % K8) * 8;
    *(u32x4*)(&k_s[t * KB + c8]) = kv[i];
    if constexpr (CAUSAL) *(u32x4*)(&q_s[t * KB + c8]) = qv[i];
    if constexpr (HAS_B) *(u32x4*)(&b_s[t * KB + c8]) = bv[i];
  }
  for (int idx = tid; idx < C * LP; idx += 256) A_s[idx] = 0.f;

  if (tid < K * TPC) {
    const int c = tid % K, seg = tid / K;
    float run = 0.f;
#pragma unroll
    for (int i = 0; i < SEG; ++i) {
      const int t = seg * SEG + i;
      if constexpr (G_CUM) {
        gk_s[t * KP + c] = gv[i];
      } else {
        run += gv[i];
        gk_s[t * KP + c] = run;
      }
    }
    if constexpr (!G_CUM) tot_s[seg * K + c] = run;
  }
  __syncthreads();
  if (tid < K * TPC) {
    const int c = tid % K, seg = tid / K;
    if constexpr (!G_CUM) {
      float off = 0.f;
      for (int s2 = 0; s2 < seg; ++s2) off += tot_s[s2 * K + c];
#pragma unroll
      for (int i = 0; i < SEG; ++i) {
        const int t = seg * SEG + i;
        gk_s[t * KP + c] = (gk_s[t * KP + c] + off) * kRcpLn2;
      }
    } else {
      // padding rows repeat the last valid cumulative decay
      const float last = gk_s[(len - 1) * KP + c];
#pragma unroll
      for (int i = 0; i < SEG; ++i) {
        const int t = seg * SEG + i;
        if (t >= len) gk_s[t * KP + c] = last;
      }
    }
  }
  __syncthreads();

  // ---- phase 2: L (and scale * Aqk) row block I = wave ----------------------
  {
    const int I = wave, n = 16 * I;
    const int r = n + (lane & 15);
    // Largest in-block decay exponent; bounded factors keep fp32 exact.
    float emax = 0.f;
    for (int c = lane; c < K; c += 64) {
      const float gn = gk_s[n * KP + c];
#pragma unroll
      for (int j = 0; j < 16; ++j) emax = fmaxf(emax, gn - gk_s[(n + j) * KP + c]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) emax = fmaxf(emax, __shfl_xor(emax, off, 64));

    if (emax <= 64.f) {
      f32x4 accL = zero4(), accQ = zero4();
#pragma unroll 4
      for (int s = 0; s < K / 4; ++s) {
        const int c = 4 * s + (lane >> 4);
        const float gr = gk_s[r * KP + c], gn = gk_s[n * KP + c];
        const float kr = (float)k_s[r * KB + c];
        const float bk = HAS_B ? kr * (float)b_s[r * KB + c] : kr;
        const float fa = fast_exp2(gr - gn);  // <= 1
        const float fb = fast_exp2(gn - gr);  // >= 1, <= 2^64
        accL = mfma_f32(bk * fa, kr * fb, accL);
        if constexpr (CAUSAL) accQ = mfma_f32((float)q_s[r * KB + c] * fa, kr * fb, accQ);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 4 * (lane >> 4) + e, j = lane & 15;
        L_s[(n + i) * LP + n + j] = (j < i) ? accL[e] : 0.f;
        if constexpr (CAUSAL) Aqk_s[(n + i) * LP + n + j] = (j <= i) ? a.scale * accQ[e] : 0.f;
      }
    } else {
      // exact pairwise products, 2^(gk_i - gk_j) with j <= i only
      for (int p = lane; p < 256; p += 64) {
        const int i = p >> 4, j = p & 15;
        float sl = 0.f, sq = 0.f;
        if (j <= i) {
          for (int c = 0; c < K; ++c) {
            const float f = fast_exp2(gk_s[(n + i) * KP + c] - gk_s[(n + j) * KP + c]);
            const float kj = (float)k_s[(n + j) * KB + c];
            const float ki = (float)k_s[(n + i) * KB + c];
            const float bki = HAS_B ? ki * (float)b_s[(n + i) * KB + c] : ki;
            sl += bki * kj * f;
            if constexpr (CAUSAL) sq += (float)q_s[(n + i) * KB + c] * kj * f;
          }
        }
        L_s[(n + i) * LP + n + j] = (j < i) ? sl : 0.f;
        if constexpr (CAUSAL) Aqk_s[(n + i) * LP + n + j] = (j <= i) ? a.scale * sq : 0.f;
      }
    }

    // off-diagonal blocks J < I, re-centred at n: both factors <= 1 (fp16 safe)
    if (I > 0) {
      f16x8 aop[K / 32];
      f16x8 qop[CAUSAL ? K / 32 : 1];
#pragma unroll
      for (int s = 0; s < K / 32; ++s) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = 32 * s + 8 * (lane >> 4) + e;
          const float fa = fast_exp2(gk_s[r * KP + c] - gk_s[n * KP + c]);
          const float kr = (float)k_s[r * KB + c];
          const float bk = HAS_B ? kr * (float)b_s[r * KB + c] : kr;
          aop[s][e] = (_Float16)(bk * fa);
          if constexpr (CAUSAL) qop[s][e] = (_Float16)((float)q_s[r * KB + c] * fa);
        }
      }
      for (int J = 0; J < I; ++J) {
        const int jr = 16 * J + (lane & 15);
        f32x4 aL = zero4(), aQ = zero4();
#pragma unroll
        for (int s = 0; s < K / 32; ++s) {
          f16x8 bop;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int c = 32 * s + 8 * (lane >> 4) + e;
            bop[e] = (_Float16)((float)k_s[jr * KB + c] * fast_exp2(gk_s[n * KP + c] - gk_s[jr * KP + c]));
          }
          aL = mfma_f16(aop[s], bop, aL);
          if constexpr (CAUSAL) aQ = mfma_f16(qop[s], bop, aQ);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = n + 4 * (lane >> 4) + e, j = 16 * J + (lane & 15);
          L_s[i * LP + j] = aL[e];
          if constexpr (CAUSAL) Aqk_s[i * LP + j] = a.scale * aQ[e];
        }
      }
    }
    // blocks above the diagonal
    for (int idx = lane; idx < 16 * C; idx += 64) {
      const int i = n + idx / C, j = idx % C;
      if (j >= n + 16) {
        L_s[i * LP + j] = 0.f;
        if constexpr (CAUSAL) Aqk_s[i * LP + j] = 0.f;
      }
    }
  }
  __syncthreads();

  // ---- phase 3: diagonal inverses (wave 0) and the elementwise operands -----
  if (wave == 0) {
    const int I = lane >> 4, j = lane & 15, n = 16 * I;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sum = (i == j) ? 1.f : 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) sum -= L_s[(n + i) * LP + n + m] * x[m];
      x[i] = sum;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) A_s[(n + i) * LP + n + j] = x[i];
  }
  {
    // kg^T P-frag (rows = K channel, red = tokens) to global, xw (col-major) to LDS.
    _Float16* kg_out = a.out.kgT + unit * (size_t)(C * K);
    for (int grp = tid; grp < K * C / 8; grp += 256) {
      const int lane_f = grp & 63, rs = grp >> 6;  // rs = rt * 2 + s
      const int s = rs & 1, rt = rs >> 1;
      const int m = 16 * rt + (lane_f & 15);
      const float glast = gk_s[(C - 1) * KP + m];
      f16x8 kgv;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int t0 = 32 * s + 16 * half + 4 * (lane_f >> 4);
        bf16x4 xwv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = t0 + e;
          const float gt = gk_s[t * KP + m];
          const float kt = (float)k_s[t * KB + m];
          const float bk = HAS_B ? kt * (float)b_s[t * KB + m] : kt;
          kgv[4 * half + e] = (_Float16)(kt * fast_exp2(glast - gt));
          xwv[e] = (__bf16)(bk * fast_exp2(gt));
        }
        *(bf16x4*)(&xw_s[m * CB + t0]) = xwv;
      }
      *(f16x8*)(kg_out + (size_t)grp * 8) = kgv;
    }
    for (int c = tid; c < K; c += 256) a.out.decay[unit * K + c] = fast_exp2(gk_s[(C - 1) * KP + c]);
    if constexpr (CAUSAL) {
      __bf16* qg_out = a.out.qg + unit * (size_t)(C * K);
      for (int grp = tid; grp < C * K / 8; grp += 256) {
        const int lane_f = grp & 63, rs = grp >> 6;  // rs = rt * (K/32) + s
        const int s = rs % (K / 32), rt = rs / (K / 32);
        const int t = 16 * rt + (lane_f & 15);
        bf16x8 qv;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int c0 = 32 * s + 16 * half + 4 * (lane_f >> 4);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            qv[4 * half + e] = (__bf16)((float)q_s[t * KB + c0 + e] * fast_exp2(gk_s[t * KP + c0 + e]));
        }
        *(bf16x8*)(qg_out + (size_t)grp * 8) = qv;
      }
    }
  }
  __syncthreads();

  // ---- phase 4: xu = beta * v (f16, column-major, aliases gk_s) and the
  //      off-diagonal inverse blocks -----------------------------------------
  _Float16* xu_s = (_Float16*)gk_s;
#pragma unroll
  for (int i = 0; i < NVL; ++i) {
    const int idx = tid + 256 * i;
    const int t = idx / V8, c8 = (idx % V8) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) xu_s[(c8 + e) * CB + t] = (_Float16)((float)vreg[i][e] * breg[i][e]);
  }
  // A_{I+d, I} for d = 1, 2, 3 (one 16x16 block per wave per stage).
#pragma unroll
  for (int d = 1; d <= 3; ++d) {
    if (wave < 4 - d) {
      const int J = wave, I = wave + d;
      // T = sum_{M=J}^{I-1} L_IM A_MJ   (standard K order)
      f32x4 T = zero4();
      for (int M = J; M < I; ++M) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int kk = 4 * s + (lane >> 4);
          const float av = L_s[(16 * I + (lane & 15)) * LP + 16 * M + kk];
          const float bv = A_s[(16 * M + kk) * LP + 16 * J + (lane & 15)];
          T = mfma_f32(av, bv, T);
        }
      }
      // R = A_II T, contracting index k = 4*(lane/16) + s so T's C layout is the B operand.
      f32x4 R = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float av = A_s[(16 * I + (lane & 15)) * LP + 16 * I + 4 * (lane >> 4) + s];
        R = mfma_f32(av, T[s], R);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
        A_s[(16 * I + 4 * (lane >> 4) + e) * LP + 16 * J + (lane & 15)] = -R[e];
    }
    __syncthreads();
  }

  // ---- phase 5: W = A xw (bf16), U = A xu (f16), row tile R = wave ----------
  {
    const int R = wave;
    bf16x8 ab[2];
    f16x8 ah[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float av = A_s[(16 * R + (lane & 15)) * LP + 32 * s + 8 * (lane >> 4) + e];
        ab[s][e] = (__bf16)av;
        ah[s][e] = (_Float16)av;
      }
    }
    // U tiles straight to global in C-frag order
    _Float16* U_out = a.out.U + unit * (size_t)(C * V);
#pragma unroll
    for (int ct = 0; ct < V / 16; ++ct) {
      f32x4 acc = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const f16x8 bv = *(const f16x8*)(&xu_s[(16 * ct + (lane & 15)) * CB + 32 * s + 8 * (lane >> 4)]);
        acc = mfma_f16(ah[s], bv, acc);
      }
      f16x4 o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = (_Float16)acc[e];
      *(f16x4*)(U_out + ((size_t)(R * (V / 16) + ct) * 64 + lane) * 4) = o4;
    }
    f32x4 wacc[K / 16];
#pragma unroll
    for (int ct = 0; ct < K / 16; ++ct) {
      wacc[ct] = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const bf16x8 bv = *(const bf16x8*)(&xw_s[(16 * ct + (lane & 15)) * CB + 32 * s + 8 * (lane >> 4)]);
        wacc[ct] = mfma_bf16(ab[s], bv, wacc[ct]);
      }
    }
    __syncthreads();  // xw_s fully consumed: reuse it as the W staging buffer
    __bf16* Wst = xw_s;
#pragma unroll
    for (int ct = 0; ct < K / 16; ++ct) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        Wst[(16 * R + 4 * (lane >> 4) + e) * KB + 16 * ct + (lane & 15)] = (__bf16)wacc[ct][e];
    }
  }
  __syncthreads();
  {
    const __bf16* Wst = xw_s;
    __bf16* W_out = a.out.W + unit * (size_t)(C * K);
    for (int grp = tid; grp < C * K / 8; grp += 256) {
      const int lane_f = grp & 63, rs = grp >> 6;
      const int s = rs % (K / 32), rt = rs / (K / 32);
      const int t = 16 * rt + (lane_f & 15);
      const int c0 = 32 * s + 4 * (lane_f >> 4);
      const bf16x4 lo = *(const bf16x4*)(&Wst[t * KB + c0]);
      const bf16x4 hi = *(const bf16x4*)(&Wst[t * KB + c0 + 16]);
      *(bf16x8*)(W_out + (size_t)grp * 8) = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    if constexpr (CAUSAL) {
      _Float16* Aqk_out = a.out.Aqk + unit * (size_t)(C * C);
      for (int grp = tid; grp < C * C / 8; grp += 256) {
        const int lane_f = grp & 63, rs = grp >> 6;
        const int s = rs & 1, rt = rs >> 1;
        const int t = 16 * rt + (lane_f & 15);
        const int j0 = 32 * s + 4 * (lane_f >> 4);
        f16x8 av;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          av[e] = (_Float16)Aqk_s[t * LP + j0 + e];
          av[4 + e] = (_Float16)Aqk_s[t * LP + j0 + 16 + e];
        }
        *(f16x8*)(Aqk_out + (size_t)grp * 8) = av;
      }
    }
    if (a.A_ref != nullptr) {
      for (int idx = tid; idx < len * C; idx += 256) {
        const int t = idx / C, j = idx % C;
        a.A_ref[((size_t)(tok0 + t) * H + h) * C + j] = (__bf16)A_s[t * LP + j];
      }
    }
  }
}

template <int K, int V, bool CAUSAL, bool HAS_B, bool G_CUM>
hipError_t launch_t(const WyArgs& a, int n_chunk, bool beta_bf16, hipStream_t stream) {
  dim3 grid(n_chunk, a.H), block(256);
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

}  // namespace

hipError_t launch_wy(const WyArgs& a, int n_chunk, int K, int V, bool causal, bool g_cumulative,
                     bool beta_bf16, hipStream_t stream) {
  if (n_chunk == 0) return hipSuccess;
  if (K == 64 && V == 64) return launch_kv<64, 64>(a, n_chunk, causal, g_cumulative, beta_bf16, stream);
  if (K == 128 && V == 128) return launch_kv<128, 128>(a, n_chunk, causal, g_cumulative, beta_bf16, stream);
  return hipErrorInvalidValue;
}

}  // namespace memt
