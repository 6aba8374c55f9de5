// Row RMSNorm arithmetic shared by every kernel that normalises a row
// (device code; included by the .hip sources).
//
// norm(x) = x / (sqrt(mean x^2) + eps) * scale, eps after the square root
// (`src/cpu/model.cpp:316-334`, `src/cpu_reference.cpp:61-98`). The sum of
// squares runs in one fixed order everywhere: thread t of a 256-thread block
// accumulates the float4 units t*4 + j*1024 (j = 0, 1, ...) with explicit
// FMAs, the 64 lanes of each wave reduce by xor-shuffles, and the four wave
// sums add in wave order. A kernel that folds the norm into a product (the
// few-row projections of decode) therefore reproduces, bit for bit, what
// the standalone norm kernel feeds the unfused product.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace evo::hip {

__device__ inline float norm_wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1)
    v += __shfl_xor(v, offset, 64);
  return v;
}

// This thread's part of the sum of squares of one float4 unit.
__device__ inline float norm_square_sum(const float4 v, float sum) {
  return fmaf(v.w, v.w, fmaf(v.z, v.z, fmaf(v.y, v.y, fmaf(v.x, v.x, sum))));
}

// Block-wide reduction of the per-thread partial sums and the denominator
// sqrt(sum / width) + eps. `partial` is 4 floats of LDS; blockDim.x == 256;
// every thread returns the same value. The caller must not reuse `partial`
// before a barrier.
__device__ inline float norm_denominator(float sum, size_t width, float eps, float *partial) {
  sum = norm_wave_sum(sum);
  if ((threadIdx.x & 63) == 0)
    partial[threadIdx.x >> 6] = sum;
  __syncthreads();
  const float total = ((partial[0] + partial[1]) + partial[2]) + partial[3];
  return sqrtf(total / static_cast<float>(width)) + eps;
}

// Denominator of one row of width % 4 == 0 read from memory, in the order
// above (any width; units past it count as zeros).
__device__ inline float row_norm_denominator(const float *__restrict__ row, size_t width,
                                             float eps, float *partial) {
  float sum = 0.0F;
  for (size_t c = threadIdx.x * 4; c < width; c += 1024)
    sum = norm_square_sum(*reinterpret_cast<const float4 *>(row + c), sum);
  return norm_denominator(sum, width, eps, partial);
}

// One normalised value (division first, as the reference), rounded on its
// own: with contraction off the product cannot fuse into whatever consumes
// it (the lo plane's y - bf16(y) would otherwise see the exact product in
// one kernel and the rounded one in another).
__device__ inline float norm_value(float x, float denominator, float scale) {
#pragma clang fp contract(off)
  return x / denominator * scale;
}

}  // namespace evo::hip
