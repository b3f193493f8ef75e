// Gate and key/query prologue of the memory block, one HBM pass.
//
// QwenMemoryBlock (models/qwen/layer.py:71-97) turns the raw projections into
// the update's inputs with six to eight eager elementwise kernels:
//   g      = -exp(s_h) * softplus(f + bias_h)            fp32   (_log_decay, :71-75)
//   sqrt_b = bf16(exp(0.5 * logsigmoid(e)))               bf16   (_write_gates, :81-84)
//   beta   = bf16(sigmoid(w))                             bf16   (:85)
//   q_hat  = bf16(q / sqrt(sum q^2 + 1e-6))               bf16   (l2norm_fwd, :92-94)
//   k_til  = bf16(f32(sqrt_b) * f32(bf16(k / sqrt(sum k^2 + 1e-6))))   (:95-96)
// Here one kernel reads each input row once and writes each output once.
// The fp32 arithmetic follows the reference's op order, with the
// transcendentals on the hardware exp2 / log2 / rcp (a few fp32 ulp), so the
// bf16 outputs agree with the reference's except where that difference moves
// a value across a bf16 rounding boundary (one bf16 ulp).
//
// Layout: a lane owns 8 consecutive channels of one (token, head) row, so
// each load and store is 16 bytes and a wave touches 1 KB of each bf16 tensor
// (D = 128: 16 lanes per row, 4 rows per wave).  The row sums for the L2
// norms are butterfly reductions over the row's lanes.

#include "common.h"
#include "gdn2_internal.h"

namespace memt {
namespace {

constexpr int kPrologueThreads = 256;

struct alignas(16) Bf16x8 {
  uint16_t v[8];
};

__device__ __forceinline__ void unpack8(const Bf16x8& p, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = bf16_bits_to_f32(p.v[i]);
}

__device__ __forceinline__ uint16_t bf16_bits(float x) {
  const __bf16 b = (__bf16)x;
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ Bf16x8 pack8(const float (&x)[8]) {
  Bf16x8 p;
#pragma unroll
  for (int i = 0; i < 8; ++i) p.v[i] = bf16_bits(x[i]);
  return p;
}

template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// One (token, head) row per LPR = D / 8 lanes.  QK: also normalise q and k
// (with k scaled by sqrt_b); otherwise write sqrt_b itself.
template <int D, bool QK>
__global__ __launch_bounds__(kPrologueThreads) void prologue_kernel(PrologueArgs a) {
  constexpr int LPR = D / 8;
  const int64_t lane_id = (int64_t)blockIdx.x * kPrologueThreads + threadIdx.x;
  const int64_t row = lane_id / LPR;
  if (row >= a.rows) return;
  const int c0 = (int)(lane_id % LPR) * 8;
  const int64_t t = row / a.H;
  const int h = (int)(row % a.H);
  const int64_t hc = (int64_t)h * D + c0;

  float f[8], bias[8], e[8], w[8];
  unpack8(*(const Bf16x8*)(a.decay + t * a.decay_stride + hc), f);
  unpack8(*(const Bf16x8*)(a.decay_bias + hc), bias);
  unpack8(*(const Bf16x8*)(a.erase + t * a.erase_stride + hc), e);
  unpack8(*(const Bf16x8*)(a.write + t * a.write_stride + hc), w);
  float q[8], k[8];
  if constexpr (QK) {
    unpack8(*(const Bf16x8*)(a.q + t * a.q_stride + hc), q);
    unpack8(*(const Bf16x8*)(a.k + t * a.k_stride + hc), k);
  }

  // -exp(s_h) is computed once per head in fp32, then multiplies the softplus.
  const float neg_rate = -gate_exp(bf16_bits_to_f32(a.decay_scale_log[h]));
  float g[8], sb[8], beta[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    g[i] = neg_rate * softplus20(f[i] + bias[i]);
    sb[i] = bf16_to_f32((__bf16)sqrt_sigmoid_bf16(e[i]));
    beta[i] = sigmoid_bf16(w[i]);
  }
  const int64_t out = row * D + c0;
  float4* gp = (float4*)(a.g_out + out);
  gp[0] = float4{g[0], g[1], g[2], g[3]};
  gp[1] = float4{g[4], g[5], g[6], g[7]};
  *(Bf16x8*)(a.beta_out + out) = pack8(beta);

  if constexpr (QK) {
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sq += q[i] * q[i];
      sk += k[i] * k[i];
    }
    sq = row_sum<LPR>(sq);
    sk = row_sum<LPR>(sk);
    const float rq = 1.f / sqrtf(sq + a.eps);
    const float rk = 1.f / sqrtf(sk + a.eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      q[i] = q[i] * rq;
      k[i] = sb[i] * bf16_to_f32((__bf16)(k[i] * rk));
    }
    *(Bf16x8*)(a.q_out + out) = pack8(q);
    *(Bf16x8*)(a.k_out + out) = pack8(k);
  } else {
    *(Bf16x8*)(a.erase_out + out) = pack8(sb);
  }
}

template <int D>
hipError_t launch_d(const PrologueArgs& a, bool qk, hipStream_t stream) {
  const int64_t lanes = a.rows * (D / 8);
  const dim3 grid((unsigned)((lanes + kPrologueThreads - 1) / kPrologueThreads)), block(kPrologueThreads);
  if (qk)
    hipLaunchKernelGGL((prologue_kernel<D, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((prologue_kernel<D, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prologue(const PrologueArgs& a, int D, bool qk, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  switch (D) {
    case 64:
      return launch_d<64>(a, qk, stream);
    case 128:
      return launch_d<128>(a, qk, stream);
    case 256:
      return launch_d<256>(a, qk, stream);
    case 512:
      return launch_d<512>(a, qk, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace memt
