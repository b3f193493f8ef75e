// Roof probes for the benchmark (libmemt_roofs.so, not part of the GDN-2
// library): a streaming read of a device buffer and a dense bf16 MFMA loop,
// the two ceilings the memory path is measured against on the GPU it runs on.
#include <hip/hip_runtime.h>
#include <stddef.h>

#include "common.h"

namespace {

constexpr int kThreads = 256;

// Every thread keeps four 16-byte non-temporal loads in flight per step and
// writes one partial sum, so nothing is dead code.  Indices stay below n4.
__global__ __launch_bounds__(kThreads) void read_probe(const memt::f32x4* __restrict__ x, size_t n4,
                                                        float* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * kThreads;
  size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  memt::f32x4 a0 = memt::f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0, a3 = a0;
  for (; i + 3 * stride < n4; i += 4 * stride) {
    a0 += __builtin_nontemporal_load(x + i);
    a1 += __builtin_nontemporal_load(x + i + stride);
    a2 += __builtin_nontemporal_load(x + i + 2 * stride);
    a3 += __builtin_nontemporal_load(x + i + 3 * stride);
  }
  for (; i < n4; i += stride) a0 += __builtin_nontemporal_load(x + i);
  const memt::f32x4 s = a0 + a1 + a2 + a3;
  out[(size_t)blockIdx.x * kThreads + threadIdx.x] = s[0] + s[1] + s[2] + s[3];
}

// Eight independent accumulator chains of v_mfma_f32_16x16x32_bf16 per wave
// (16384 flop each), started from distinct values so no two chains fold into
// one; operands come from the thread index.
constexpr int kChains = 8;
__global__ __launch_bounds__(kThreads) void mfma_probe(int iters, float* __restrict__ out) {
  memt::bf16x8 a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (__bf16)(1.f + 1e-3f * (float)((threadIdx.x + j) & 7));
    b[j] = (__bf16)(1.f - 1e-3f * (float)((threadIdx.x + 3 * j) & 7));
  }
  memt::f32x4 c[kChains];
#pragma unroll
  for (int j = 0; j < kChains; ++j) {
    // a splat start value keeps each chain in one register tuple across the loop
    const float v0 = (float)(j + threadIdx.x);
    c[j] = memt::f32x4{v0, v0, v0, v0};
  }
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < kChains; ++j) c[j] = memt::mfma_bf16(a, b, c[j]);
  }
  // every accumulator is stored, so no chain can be dropped as dead code
  memt::f32x4* o = (memt::f32x4*)out + ((size_t)blockIdx.x * kThreads + threadIdx.x) * kChains;
#pragma unroll
  for (int j = 0; j < kChains; ++j) o[j] = c[j];
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16, 16-byte aligned) of x; out holds blocks * 256 floats.
int memt_roofs_read(const void* x, size_t bytes, float* out, int blocks, hipStream_t stream) {
  if (x == nullptr || out == nullptr || blocks <= 0 || bytes % 16 != 0 || ((uintptr_t)x & 15) != 0) return -1;
  hipLaunchKernelGGL(read_probe, dim3(blocks), dim3(kThreads), 0, stream, (const memt::f32x4*)x, bytes / 16, out);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// blocks * 4 waves each run kChains * iters MFMAs of 16384 flop; out holds
// blocks * 256 * kChains * 4 floats (every accumulator of every lane).
int memt_roofs_mfma(float* out, int blocks, int iters, hipStream_t stream) {
  if (out == nullptr || blocks <= 0 || iters <= 0) return -1;
  hipLaunchKernelGGL(mfma_probe, dim3(blocks), dim3(kThreads), 0, stream, iters, out);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

}  // extern "C"
