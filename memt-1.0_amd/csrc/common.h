// Shared device helpers for the GDN-2 memory kernels (gfx950 / CDNA4, wave64).
//
// MFMA lane layouts used throughout (checked on gfx950 against a host matmul):
//   v_mfma_f32_16x16x32_{bf16,f16}: A[16x32]: lane l holds A[l%16][8*(l/16) + 0..7]
//                                    B[32x16]: lane l holds B[8*(l/16) + 0..7][l%16]
//                                    C[16x16]: lane l holds C[4*(l/16) + 0..3][l%16]
//   v_mfma_f32_16x16x4_f32:          A: lane l holds A[l%16][l/16]; B: B[l/16][l%16]; C as above.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace memt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 1/ln(2) as the reference's cumsum scale (FLA/ops/utils/constant.py:10).
constexpr float kRcpLn2 = 1.4426950216f;

__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f16(const f16x8& a, const f16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One direct load (global_load_lds_dwordx4): lane l's 16 bytes at src_lane land
// at dst + 16 l (dst uniform over the wave, 16-byte aligned).  Written as inline
// assembly so that the compiler does not see an LDS write in flight and wait for
// it before every later LDS read: the caller waits for these loads itself
// (s_waitcnt vmcnt) before the barrier that precedes their use.  M0, the LDS base
// of the load (one wait state between its write and the load), is set for each
// load: a kernel that calls this must use M0 for nothing else (M0 is reserved to
// the compiler, so it cannot be declared clobbered).
__device__ __forceinline__ void lds_dma16(const void* src_lane, char* dst) {
  const unsigned lds_addr = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)dst);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src_lane), "s"(lds_addr)
               : "memory");
}

// Native v_exp_f32 (base 2).  Inputs below -126 give denormal/zero results.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Gate transcendentals on the hardware exp2 / log2 / rcp, a few fp32 ulp from
// the correctly rounded values (the gates' bf16 outputs round that away).
// exp(x) = 2^(x log2 e): the product is carried as hi + lo (log2 e split in
// two fp32 parts, fma for the rounding of x * hi), and 2^lo ~ 1 + lo ln 2.
__device__ __forceinline__ float gate_exp(float x) {
  constexpr float kL2eHi = 1.44269502f, kL2eLo = 1.92596299e-8f, kLn2 = 0.693147182f;
  const float p = x * kL2eHi;
  const float lo = fmaf(x, kL2eHi, -p) + x * kL2eLo;
  return __builtin_amdgcn_exp2f(p) * fmaf(lo, kLn2, 1.f);
}
// log1p(y) for y >= 0: log(u) * y / (u - 1) with u = 1 + y, which cancels the
// rounding of u (D. Goldberg, "What every computer scientist should know about
// floating-point arithmetic", 1991, Theorem 4).
__device__ __forceinline__ float gate_log1p(float y) {
  const float u = 1.f + y;
  if (u == 1.f) return y;
  return __builtin_amdgcn_logf(u) * 0.693147182f * (y * __builtin_amdgcn_rcpf(u - 1.f));
}
// torch.nn.functional.softplus (beta 1, threshold 20), as max(x, 0) + log1p(e^-|x|)
__device__ __forceinline__ float softplus20(float x) {
  return x > 20.f ? x : fmaxf(x, 0.f) + gate_log1p(gate_exp(-fabsf(x)));
}
// torch.nn.functional.logsigmoid: min(x, 0) - log1p(e^-|x|)
__device__ __forceinline__ float logsigmoid(float x) { return fminf(x, 0.f) - gate_log1p(gate_exp(-fabsf(x))); }
__device__ __forceinline__ float gate_sigmoid(float x) { return __builtin_amdgcn_rcpf(1.f + gate_exp(-x)); }
// Gates whose results are stored as bf16 (beta, sqrt_b) need only ~1e-6
// relative accuracy, far below a bf16 ulp (2^-8): the plain 2^(x log2 e).
__device__ __forceinline__ float sigmoid_bf16(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.44269502f));
}
// softplus for a decay that only feeds the in-kernel cumsum: max(x, 0) +
// ln2 * log2(1 + 2^(-|x| log2 e)), absolute error ~1e-7 (the decay factors it
// yields move by ~1e-5 relative over a 64-token chunk)
__device__ __forceinline__ float softplus_internal(float x) {
  const float y = __builtin_amdgcn_exp2f(-fabsf(x) * 1.44269502f);
  return fmaxf(x, 0.f) + __builtin_amdgcn_logf(1.f + y) * 0.693147182f;
}
// sqrt_b = exp(logsigmoid(e) / 2), computed as sqrt(sigmoid(e)) (the same value)
__device__ __forceinline__ float sqrt_sigmoid_bf16(float x) { return __builtin_sqrtf(sigmoid_bf16(x)); }

__device__ __forceinline__ float bf16_to_f32(__bf16 x) { return (float)x; }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Round-to-nearest-even float -> bf16 (the conversion torch and Triton use).
__device__ __forceinline__ __bf16 f32_to_bf16(float x) { return (__bf16)x; }

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

template <typename T>
__device__ __forceinline__ float load_as_f32(const T* p);
template <>
__device__ __forceinline__ float load_as_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_as_f32<__bf16>(const __bf16* p) { return (float)*p; }

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load and store of the wave (vmcnt(0)).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// x from lane (i - N) of the same 16-lane row, 0 for the first N lanes of a row.
template <int N>
__device__ __forceinline__ float dpp_row_shr(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x110 + N, 0xF, 0xF, true));
}
// Inclusive prefix sum over the 16 lanes of each row.
__device__ __forceinline__ float row_inclusive_scan(float x) {
  x += dpp_row_shr<1>(x);
  x += dpp_row_shr<2>(x);
  x += dpp_row_shr<4>(x);
  x += dpp_row_shr<8>(x);
  return x;
}

// Max over the 16 lanes of each row for non-negative x, in lane 15 of the row
// (row-shift DPP steps shift in 0 at the row start); VALU only, no LDS traffic.
__device__ __forceinline__ float row_max_nonneg(float x) {
  x = fmaxf(x, dpp_row_shr<1>(x));
  x = fmaxf(x, dpp_row_shr<2>(x));
  x = fmaxf(x, dpp_row_shr<4>(x));
  x = fmaxf(x, dpp_row_shr<8>(x));
  return x;
}

// Wave64 sum reduction (all lanes receive the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace memt
