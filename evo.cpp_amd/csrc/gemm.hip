// SPDX-License-Identifier: Apache-2.0
// Dense linears of the StripedHyena2 block on gfx950 MFMA.
//
//   C[M,N] = A[M,K] . W[N,K]^T  (+ fused epilogue)
//
// A is the F32 activation (row-major), W the BF16 weight in nn.Linear layout
// ([out, in], K contiguous), accumulation F32. Reference semantics: the
// F32-activation x BF16-weight dot of evo.cpp `src/cpu/model.cpp:284-314`.
//
// Precision: in the "split" variant each F32 activation is written as
// hi + lo with hi = bf16(a) and lo = bf16(a - hi); both halves are multiplied
// by the (exactly BF16) weight on MFMA, so the product carries ~16 significant
// bits of the activation (relative error ~2^-17) for twice the MFMA work. The
// "bf16" variant keeps only hi (one MFMA pass).
//
// Tiling for CDNA4: 256 threads = 4 waves; block tile 128x128, K step 32;
// each wave owns a 64x64 sub-tile = 2x2 MFMA 32x32x16 tiles (64 F32
// accumulators per lane). Global loads are 16-byte vectors, staged through
// LDS rows padded to 40 BF16 (80 B) so the 16-byte per-lane fragment reads of
// 32 consecutive rows spread over the banks. The next K tile is fetched into
// registers while the current one is multiplied.
#include "common.hpp"
#include "ops.hpp"

namespace evo::hip {
namespace {

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 32;
constexpr int kLdsStride = kBK + 8;  // BF16 elements per LDS row

struct Epilogue {
  int mode;              // GemmEpilogue
  const uint16_t *bias;  // BF16 [N] (bias modes)
  const float *residual; // F32 [M, ldc] (residual modes)
  int gelu;              // gated mode: 1 = erf-GELU on the l1 half
  int gated_width;       // gated mode: number of valid output columns
};

__device__ inline float gelu_erf(const float x) {
  return 0.5F * x * (1.0F + erff(x * 0.7071067811865475244F));
}

template <bool kSplit>
__global__ __launch_bounds__(256) void gemm_bf16w_kernel(
    const float *__restrict__ A, const uint16_t *__restrict__ W,
    float *__restrict__ C, const int M, const int N, const int K,
    const int ldc, const Epilogue epi) {
  __shared__ __attribute__((aligned(16))) uint16_t a_hi[kBM * kLdsStride];
  __shared__ __attribute__((aligned(16))) uint16_t a_lo[kSplit ? kBM * kLdsStride : 8];
  __shared__ __attribute__((aligned(16))) uint16_t w_s[kBN * kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_m = wave >> 1;
  const int wave_n = wave & 1;
  const int block_m = blockIdx.y * kBM;
  const int block_n = blockIdx.x * kBN;

  // Loader mapping: thread -> (row, 16-element K segment).
  const int load_row = tid >> 1;
  const int load_k = (tid & 1) * 16;
  const int a_row = block_m + load_row;
  const int w_row = block_n + load_row;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[i][j][e] = 0.0F;

  float a_reg[16];
  uint4 w_reg[2];

  auto fetch = [&](const int k0) {
    const int k = k0 + load_k;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float4 value = make_float4(0.F, 0.F, 0.F, 0.F);
      if (a_row < M && k + v * 4 < K)
        value = *reinterpret_cast<const float4 *>(A + static_cast<size_t>(a_row) * K + k + v * 4);
      a_reg[v * 4 + 0] = value.x;
      a_reg[v * 4 + 1] = value.y;
      a_reg[v * 4 + 2] = value.z;
      a_reg[v * 4 + 3] = value.w;
    }
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      uint4 value = make_uint4(0U, 0U, 0U, 0U);
      if (w_row < N && k + v * 8 < K)
        value = *reinterpret_cast<const uint4 *>(W + static_cast<size_t>(w_row) * K + k + v * 8);
      w_reg[v] = value;
    }
  };

  auto stash = [&]() {
    uint32_t hi[8], lo[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const float x0 = a_reg[2 * p], x1 = a_reg[2 * p + 1];
      const uint16_t h0 = f32_to_bf16(x0), h1 = f32_to_bf16(x1);
      hi[p] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16U);
      if (kSplit) {
        const uint16_t l0 = f32_to_bf16(x0 - bf16_to_f32(h0));
        const uint16_t l1 = f32_to_bf16(x1 - bf16_to_f32(h1));
        lo[p] = static_cast<uint32_t>(l0) | (static_cast<uint32_t>(l1) << 16U);
      }
    }
    uint4 *dst_hi = reinterpret_cast<uint4 *>(a_hi + load_row * kLdsStride + load_k);
    dst_hi[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    dst_hi[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    if (kSplit) {
      uint4 *dst_lo = reinterpret_cast<uint4 *>(a_lo + load_row * kLdsStride + load_k);
      dst_lo[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
      dst_lo[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
    }
    uint4 *dst_w = reinterpret_cast<uint4 *>(w_s + load_row * kLdsStride + load_k);
    dst_w[0] = w_reg[0];
    dst_w[1] = w_reg[1];
  };

  fetch(0);
  for (int k0 = 0; k0 < K; k0 += kBK) {
    __syncthreads();
    stash();
    __syncthreads();
    if (k0 + kBK < K)
      fetch(k0 + kBK);
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      const int koff = ks + (lane >> 5) * 8;
      bf16x8 bh[2], bl_unused;
      (void)bl_unused;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = wave_n * 64 + j * 32 + (lane & 31);
        bh[j] = *reinterpret_cast<const bf16x8 *>(w_s + col * kLdsStride + koff);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wave_m * 64 + i * 32 + (lane & 31);
        const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(a_hi + row * kLdsStride + koff);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh[j], acc[i][j], 0, 0, 0);
        if (kSplit) {
          const bf16x8 al = *reinterpret_cast<const bf16x8 *>(a_lo + row * kLdsStride + koff);
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh[j], acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // Epilogue. Accumulator e of tile (i, j): row i*32 + (e/4)*8 + (lane/32)*4 + e%4,
  // column j*32 + lane%32 of the wave's 64x64 sub-tile.
  const int col_base = block_n + wave_n * 64 + (lane & 31);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = block_m + wave_m * 64 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
      if (row >= M)
        continue;
      if (epi.mode == kGemmGated) {
        // Columns [64q, 64q+32) hold l1 rows, [64q+32, 64q+64) the matching l2
        // rows, so one lane owns both operands of its gated output.
        const int out_col = (block_n + wave_n * 64) / 2 + (lane & 31);
        if (out_col < epi.gated_width) {
          const float first = acc[i][0][e];
          const float activated = epi.gelu ? gelu_erf(first) : first;
          C[static_cast<size_t>(row) * ldc + out_col] = activated * acc[i][1][e];
        }
        continue;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int col = col_base + j * 32;
        if (col >= N)
          continue;
        float value = acc[i][j][e];
        const size_t index = static_cast<size_t>(row) * ldc + col;
        if (epi.mode == kGemmBiasResidual) {
          value = value + bf16_to_f32(epi.bias[col]);
          value = value + epi.residual[index];
        } else if (epi.mode == kGemmResidual) {
          value = value + epi.residual[index];
        } else if (epi.mode == kGemmBias) {
          value = value + bf16_to_f32(epi.bias[col]);
        }
        C[index] = value;
      }
    }
  }
}

}  // namespace

Status gemm_bf16w(const float *A, const uint16_t *W, float *C, size_t M,
                  size_t N, size_t K, size_t ldc, GemmEpilogue mode,
                  const uint16_t *bias, const float *residual, bool gelu,
                  size_t gated_width, bool split, hipStream_t stream) {
  if (A == nullptr || W == nullptr || C == nullptr || M == 0 || N == 0 ||
      K == 0 || K % 8 != 0 || M > (1U << 30) || N > (1U << 30) ||
      K > (1U << 30))
    return {ErrorCode::kInvalidArgument,
            "gemm_bf16w: null operand or unsupported shape (K must be a positive multiple of 8)"};
  if ((mode == kGemmBias || mode == kGemmBiasResidual) && bias == nullptr)
    return {ErrorCode::kInvalidArgument, "gemm_bf16w: bias epilogue needs a bias"};
  if ((mode == kGemmResidual || mode == kGemmBiasResidual) && residual == nullptr)
    return {ErrorCode::kInvalidArgument, "gemm_bf16w: residual epilogue needs a residual"};
  if (mode == kGemmGated && (N % 64 != 0 || gated_width * 2 > N))
    return {ErrorCode::kInvalidArgument,
            "gemm_bf16w: gated epilogue needs N = 2*padded width, multiple of 64"};
  if (mode != kGemmGated && ldc < N)
    return {ErrorCode::kInvalidArgument, "gemm_bf16w: ldc < N"};
  Epilogue epi{static_cast<int>(mode), bias, residual, gelu ? 1 : 0,
               static_cast<int>(gated_width)};
  const dim3 grid(ceil_div(N, kBN), ceil_div(M, kBM));
  if (split)
    hipLaunchKernelGGL(gemm_bf16w_kernel<true>, grid, dim3(256), 0, stream, A, W, C,
                       static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                       static_cast<int>(ldc), epi);
  else
    hipLaunchKernelGGL(gemm_bf16w_kernel<false>, grid, dim3(256), 0, stream, A, W, C,
                       static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                       static_cast<int>(ldc), epi);
  return launch_status("gemm_bf16w_kernel");
}

}  // namespace evo::hip
