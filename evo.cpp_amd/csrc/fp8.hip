// SPDX-License-Identifier: Apache-2.0
// Software-FP8 projection executor on gfx950.
//
// Quantiser: code = E4M3FN(float(bf16(x)) * scale), round to nearest even,
// saturating finite overflow and infinities to +-448, NaN -> 0x7f|sign, sign
// kept on values rounding to zero. This is the code set of evo.cpp
// `src/fp8.cpp:26-58` (the reference searches the code table; here the code is
// computed from the binade: subnormals as rint(m * 2^9), normals as
// rint(m * 2^(3-e)) offset by the exponent field, which yields the same code
// including tie-to-even on the code's low bit). Applied to BF16 activations
// as in `src/cuda/ops.cu:250-262`.
//
// GEMM, three modes over E4M3 codes A [M,K] and W [N,K]:
//  * exact: the integer QGMMA emulation of `src/cuda/ops.cu:277-441` -- per
//    K=32 group the maximum exponent over the accumulator and all nonzero
//    products, every term aligned to 13 fractional bits and truncated, one
//    integer sum, E8M13 truncation of the normalised result;
//  * mfma-k32 / mfma-k128: OCP-E4M3 MFMA (v_mfma_f32_32x32x16_fp8_fp8 or
//    v_mfma_scale_f32_32x32x64_f8f6f4 with unit scales) adds each K chunk's
//    products onto the running accumulator in F32, which is then truncated
//    to E8M13 like the reference's after every group. Per-term truncation
//    inside a chunk is not reproduced, so results differ from exact mode by
//    a few E8M13 ulps.
// All modes finish with bf16(acc * output_scale).
#include <type_traits>

#include "common.hpp"
#include "row_norm.hpp"
#include "ops.hpp"

namespace evo::hip {
namespace {


__global__ void quantize_f32_kernel(const float *__restrict__ x, size_t n,
                                    float scale, uint8_t *__restrict__ codes) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
       i < n; i += static_cast<size_t>(gridDim.x) * blockDim.x)
    codes[i] = encode_e4m3(round_bf16(x[i]) * scale);
}

__global__ void quantize_bf16_kernel(const uint16_t *__restrict__ x, size_t n,
                                     float scale, uint8_t *__restrict__ codes) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
       i < n; i += static_cast<size_t>(gridDim.x) * blockDim.x)
    codes[i] = encode_e4m3(bf16_to_f32(x[i]) * scale);
}

// Packed integer form of a code: 4-bit significand (bits 0-4), exponent + 16
// (bits 5-9), sign (bit 10); value = significand/8 * 2^exponent.
__device__ inline uint16_t pack_code(const uint8_t code) {
  const unsigned field = (code >> 3U) & 0x0fU;
  const unsigned mantissa = code & 0x07U;
  int exponent;
  unsigned significand;
  if (field == 0U) {
    if (mantissa == 0U)
      return 0U;
    const int lead = 31 - __clz(mantissa);
    exponent = lead - 9;
    significand = mantissa << (3 - lead);
  } else {
    exponent = static_cast<int>(field) - 7;
    significand = 8U + mantissa;
  }
  return static_cast<uint16_t>(significand | ((exponent + 16) << 5) |
                               ((code & 0x80U) ? 0x400U : 0U));
}

__device__ inline float truncate_e8m13(const float v) {
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & 0xfffffc00U);
}

__device__ inline int float_exponent(const float v) {
  return static_cast<int>((__builtin_bit_cast(uint32_t, v) >> 23U) & 0xffU) - 127;
}

// Exact QGMMA: 16x16 outputs per 256-thread block, one output per thread.
constexpr int kExactTile = 16;
constexpr int kGroup = 32;

template <typename Out>
__global__ __launch_bounds__(256) void qgmma_exact_kernel(
    const uint8_t *__restrict__ a, const uint8_t *__restrict__ w,
    Out *__restrict__ out, int M, int N, int K, float output_scale) {
  __shared__ uint16_t a_tile[kExactTile][kGroup];
  __shared__ uint16_t w_tile[kGroup][kExactTile + 1];
  const int t = threadIdx.x;
  const int lr = t / kExactTile, lc = t % kExactTile;
  const int row = blockIdx.y * kExactTile + lr;
  const int col = blockIdx.x * kExactTile + lc;
  float acc = 0.0F;
  for (int k0 = 0; k0 < K; k0 += kGroup) {
    for (int i = t; i < kExactTile * kGroup; i += 256) {
      const int r = i / kGroup, k = i % kGroup;
      const int gr = blockIdx.y * kExactTile + r;
      const int gc = blockIdx.x * kExactTile + r;
      a_tile[r][k] = gr < M ? pack_code(a[static_cast<size_t>(gr) * K + k0 + k]) : 0;
      w_tile[k][r] = gc < N ? pack_code(w[static_cast<size_t>(gc) * K + k0 + k]) : 0;
    }
    __syncthreads();
    int top = acc == 0.0F ? -1024 : float_exponent(acc);
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      const uint16_t l = a_tile[lr][k], r = w_tile[k][lc];
      if ((l & 0x1fU) && (r & 0x1fU))
        top = max(top, static_cast<int>((l >> 5) & 0x1fU) +
                           static_cast<int>((r >> 5) & 0x1fU) - 32);
    }
    int32_t sum = 0;
    if (acc != 0.0F) {
      const uint32_t bits = __builtin_bit_cast(uint32_t, acc);
      uint32_t significand = ((bits & 0x7fffffU) | 0x800000U) >> 10U;
      const int shift = top - float_exponent(acc);
      significand = shift > 31 ? 0U : (significand >> shift);
      sum = (bits & 0x80000000U) ? -static_cast<int32_t>(significand)
                                 : static_cast<int32_t>(significand);
    }
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      const uint16_t l = a_tile[lr][k], r = w_tile[k][lc];
      if ((l & 0x1fU) && (r & 0x1fU)) {
        const int shift = top - (static_cast<int>((l >> 5) & 0x1fU) +
                                 static_cast<int>((r >> 5) & 0x1fU) - 32);
        if (shift <= 31) {
          const uint32_t value = ((l & 0x1fU) * (r & 0x1fU) * 128U) >> shift;
          sum += ((l ^ r) & 0x400U) ? -static_cast<int32_t>(value)
                                    : static_cast<int32_t>(value);
        }
      }
    }
    acc = sum == 0 ? 0.0F : truncate_e8m13(ldexpf(static_cast<float>(sum), top - 13));
    __syncthreads();
  }
  if (row < M && col < N)
    put(out, static_cast<size_t>(row) * N + col, round_bf16(acc * output_scale));
}

// MFMA path. Block 128 (M) x 192 (N) outputs, 4 waves as 2 (M) x 2 (N) of
// 64 x 96 (2 x 3 MFMA 32x32 tiles); two blocks share a CU (80 KB of LDS
// each), so two waves per SIMD and one block's barrier wait runs under the
// other block's MFMAs; the 96 accumulators
// per lane stay in VGPRs, so the E8M13 truncation after each promotion is
// one VALU op per value. The accumulator is the MFMA's C operand: a chunk's
// products are summed onto it inside the matrix core and the sum is
// truncated (the reference also adds the aligned accumulator into each
// group's integer sum). K is staged 128 codes (one 128-byte line per row)
// per step by DMA into LDS rows of eight 16-byte units, unit u of row r at
// r*8 + (u ^ ((r >> 1) & 7)) so that the fragment reads of 8 consecutive rows
// hit 8 distinct bank groups; two stages alternate. A 1024-row projection
// is 8 x 64 = 512 tiles: two per CU. Rows beyond M or N load a clamped
// valid row and are never stored.
constexpr int kBM = 128, kBN = 192, kBK = 128, kStages = 2;
constexpr int kWaves = 4;
constexpr int kStageBytes = (kBM + kBN) * kBK;            // 40 KB
constexpr int kDmaPerWave = kStageBytes / 1024 / kWaves;  // 10
constexpr size_t kMfmaLds = static_cast<size_t>(kStages) * kStageBytes;

__device__ inline int fp8_unit(int row, int unit) { return row * 8 + (unit ^ ((row >> 1) & 7)); }

template <int kChunk, typename Out>
__global__ __launch_bounds__(kWaves * 64, 2) void fp8_mfma_kernel(
    const uint8_t *__restrict__ a, const uint8_t *__restrict__ w,
    Out *__restrict__ out, int M, int N, int K, float output_scale) {
  extern __shared__ __attribute__((aligned(16))) uint8_t fp8_lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, col = lane & 31;
  const int wave_m = wave >> 1, wave_n = wave & 1;  // 2 x 2
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  const int block_m = tm * kBM, block_n = tn * kBN;

  // DMA op g = wave*10 + i: 1 KB chunk g of the stage (chunks 0..15 = A rows
  // 8g.., 16..39 = W rows 8(g-16)..); lane l fills unit 64 g' + l. Each op
  // reads from a wave-uniform base (the block's first A or W row, advanced
  // by the step's K offset) plus a fixed 32-bit per-lane offset.
  const uint8_t *a_base = a + static_cast<size_t>(block_m) * K;
  const uint8_t *w_base = w + static_cast<size_t>(block_n) * K;
  uint32_t src[kDmaPerWave];
  int dst[kDmaPerWave];
  bool from_a[kDmaPerWave];
#pragma unroll
  for (int i = 0; i < kDmaPerWave; ++i) {
    const int g = wave * kDmaPerWave + i;
    const bool is_a = g < kBM / 8;
    const int chunk = is_a ? g : g - kBM / 8;
    const int flat = chunk * 64 + lane;
    const int row = flat >> 3, unit = (flat & 7) ^ ((row >> 1) & 7);
    const int clamped = is_a ? min(block_m + row, M - 1) - block_m
                             : min(block_n + row, N - 1) - block_n;
    src[i] = static_cast<uint32_t>(clamped) * static_cast<uint32_t>(K) + unit * 16;
    dst[i] = (is_a ? 0 : kBM * kBK) + chunk * 1024;
    from_a[i] = is_a;
  }
  auto issue = [&](int step) {
    uint8_t *stage = fp8_lds + (step % kStages) * kStageBytes;
    const int k0 = step * kBK;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i)
      dma16((from_a[i] ? a_base : w_base) + k0, src[i], stage + dst[i]);
  };

  f32x16 acc[2][3];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[i][j][e] = 0.0F;
  auto frag32 = [&](const uint8_t *base, int row, int unit) {
    const uint4 lo = *reinterpret_cast<const uint4 *>(base + fp8_unit(row, unit) * 16);
    const uint4 hi = *reinterpret_cast<const uint4 *>(base + fp8_unit(row, unit + 1) * 16);
    return i32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                 (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  };

  const int steps = K / kBK;
  issue(0);
  for (int s = 0; s < steps; ++s) {
    wait_dma<0>();
    // Every wave's DMA of step s has landed and every wave has left the
    // buffer of step s-1, which the next issue overwrites.
    __syncthreads();
    const uint8_t *a_s = fp8_lds + (s % kStages) * kStageBytes;
    const uint8_t *w_s = a_s + kBM * kBK;
    if constexpr (kChunk == 128) {
      // Two K=64 MFMAs per tile, then one promotion (truncation) per 128 K.
      i32x8 av[2][2], bv[2][3];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int j = 0; j < 3; ++j)
          bv[ks][j] = frag32(w_s, wave_n * 96 + j * 32 + col, ks * 4 + half * 2);
#pragma unroll
        for (int i = 0; i < 2; ++i)
          av[ks][i] = frag32(a_s, wave_m * 64 + i * 32 + col, ks * 4 + half * 2);
      }
      // The next step's DMA (into the buffer of step s-1, which every wave
      // has left) goes out behind the fragment reads and ahead of the MFMAs:
      // placed between the two K halves instead it measured 3 % slower
      // (config 3: 54.5 -> 56 us; M = 8192: 420 -> 435 us, bit-identical).
      if (s + 1 < steps)
        issue(s + 1);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
              av[0][i], bv[0][j], acc[i][j], 0, 0, 0, 127, 0, 127);
      // Second K half: each tile's promotion runs while the next tile's
      // MFMA executes (only the last tile's truncation is left at the end).
#pragma unroll
      for (int t = 0; t < 6; ++t) {
        const int i = t / 3, j = t % 3;
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            av[1][i], bv[1][j], acc[i][j], 0, 0, 0, 127, 0, 127);
        if (t > 0) {
          const int pi = (t - 1) / 3, pj = (t - 1) % 3;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            acc[pi][pj][e] = truncate_e8m13(acc[pi][pj][e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[1][2][e] = truncate_e8m13(acc[1][2][e]);
    } else {
      // Four 32-K chunks, each two K=16 MFMAs per tile then a promotion.
      // A tile's promotion is issued right behind the next tile's second
      // MFMA, so the truncations run under the matrix core's work instead
      // of after it; the last tile's promotion waits until just before its
      // first MFMA of the next chunk (same values: each truncation still
      // sits between the chunk that produced it and the next one).
#pragma unroll
      for (int c = 0; c < kBK / 32; ++c) {
        // Lane half h reads the 16 codes [32c + 16h, 32c + 16h + 16) of its
        // row in one 16-byte read (the conflict-free pattern of the K128
        // path; two 8-byte reads per chunk put rows r and r + 16 on the same
        // banks): the chunk's first MFMA takes codes 0-7 of each half, the
        // second codes 8-15. A and W are split the same way, so the chunk
        // still sums exactly its 32 products before the promotion.
        long bv[2][3], av[2][2];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const int row = wave_n * 96 + j * 32 + col;
          const uint4 v = *reinterpret_cast<const uint4 *>(w_s + fp8_unit(row, 2 * c + half) * 16);
          bv[0][j] = static_cast<long>((static_cast<unsigned long>(v.y) << 32) | v.x);
          bv[1][j] = static_cast<long>((static_cast<unsigned long>(v.w) << 32) | v.z);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int row = wave_m * 64 + i * 32 + col;
          const uint4 v = *reinterpret_cast<const uint4 *>(a_s + fp8_unit(row, 2 * c + half) * 16);
          av[0][i] = static_cast<long>((static_cast<unsigned long>(v.y) << 32) | v.x);
          av[1][i] = static_cast<long>((static_cast<unsigned long>(v.w) << 32) | v.z);
        }
#pragma unroll
        for (int t = 0; t < 6; ++t) {
          if (t == 5) {  // truncating the initial zeros is harmless
#pragma unroll
            for (int e = 0; e < 16; ++e)
              acc[1][2][e] = truncate_e8m13(acc[1][2][e]);
          }
          acc[t / 3][t % 3] = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(
              av[0][t / 3], bv[0][t % 3], acc[t / 3][t % 3], 0, 0, 0);
        }
        if (c == 0 && s + 1 < steps)
          issue(s + 1);  // the next step's DMA, after the first chunk's reads
#pragma unroll
        for (int t = 0; t < 6; ++t) {
          acc[t / 3][t % 3] = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(
              av[1][t / 3], bv[1][t % 3], acc[t / 3][t % 3], 0, 0, 0);
          if (t > 0) {
            const int pi = (t - 1) / 3, pj = (t - 1) % 3;
#pragma unroll
            for (int e = 0; e < 16; ++e)
              acc[pi][pj][e] = truncate_e8m13(acc[pi][pj][e]);
          }
        }
      }
    }
  }
  if constexpr (kChunk == 32) {
    // The last chunk's deferred promotion of the last tile.
#pragma unroll
    for (int e = 0; e < 16; ++e)
      acc[1][2][e] = truncate_e8m13(acc[1][2][e]);
  }
  if constexpr (std::is_same<Out, uint16_t>::value) {
    if (N % 2 == 0 && reinterpret_cast<uintptr_t>(out) % 4 == 0) {
      // BF16 pairs: lanes col and col ^ 1 swap one value of each row pair
      // (e, e + 1), so the even lane stores row r at columns (col, col + 1)
      // and the odd lane row r + 1 at (col - 1, col): one 32-bit store per
      // two values.
      const bool even = (col & 1) == 0;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const int row = block_m + wave_m * 64 + i * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
#pragma unroll
          for (int j = 0; j < 3; ++j) {
            const uint32_t first = f32_to_bf16(round_bf16(acc[i][j][e] * output_scale));
            const uint32_t second = f32_to_bf16(round_bf16(acc[i][j][e + 1] * output_scale));
            const uint32_t other = static_cast<uint32_t>(__shfl_xor(
                static_cast<int>(even ? second : first), 1, 64));
            const int out_row = even ? row : row + 1;
            const int column = block_n + wave_n * 96 + j * 32 + (col & ~1);
            if (out_row < M && column < N)
              *reinterpret_cast<uint32_t *>(out + static_cast<size_t>(out_row) * N + column) =
                  even ? (first | (other << 16)) : (other | (second << 16));
          }
        }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = block_m + wave_m * 64 + i * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
      if (row >= M)
        continue;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int column = block_n + wave_n * 96 + j * 32 + col;
        if (column < N)
          put(out, static_cast<size_t>(row) * N + column,
              round_bf16(acc[i][j][e] * output_scale));
      }
    }
}

// ---- Few-row projection (decode, M <= 4, MFMA modes): each 256-thread
// block owns 8 weight rows, wave w the rows 2w and 2w+1 over all of K; lane
// l reads 16 codes of a row per 1024-K sweep. Codes decode to F32 (the
// hardware OCP-E4M3 convert), products are exact, and the lanes of one
// kChunk-K group sum their partials by shuffles; the group sums go to LDS
// and one thread per (row, activation row) then promotes them in K order,
// acc = trunc_E8M13(acc + chunk), finishing with bf16(acc * output_scale).
// The activation codes of the block's rows are decoded into LDS once.
constexpr int kGemv8Rows = 16;
constexpr int kGemv8MaxM = 4;
constexpr int kGemv8MaxK = 8192;

typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ inline void decode16(const uint4 codes, float (&out)[16]) {
  const unsigned words[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(words[q]), false);
    const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(words[q]), true);
    out[4 * q] = lo.x;
    out[4 * q + 1] = lo.y;
    out[4 * q + 2] = hi.x;
    out[4 * q + 3] = hi.y;
  }
}

template <int kChunk, int kM, typename Out>
__global__ __launch_bounds__(256) void fp8_gemv_kernel(
    const uint8_t *__restrict__ a, const uint8_t *__restrict__ w, Out *__restrict__ out,
    int M, int N, int K, float output_scale, const RowNorm norm, float code_scale) {
  constexpr int kLanesPerChunk = kChunk / 16;
  constexpr int kRowsPerWave = kGemv8Rows / 4;
  // LDS: chunk sums [kGemv8Rows][M][K/kChunk], then (folded norm) the
  // activation codes [M][K].
  extern __shared__ float chunk_s[];
  __shared__ float norm_partial[4];
  const int chunks = K / kChunk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * kGemv8Rows + wave * kRowsPerWave;
  // The codes of the next 1024-K sweep load before this sweep is multiplied.
  auto load_codes = [&](int k, uint4 (&codes)[kRowsPerWave]) {
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
      codes[r] = row0 + r < N ? *reinterpret_cast<const uint4 *>(
                                    w + static_cast<size_t>(row0 + r) * K + k)
                              : make_uint4(0, 0, 0, 0);
  };
  int k = lane * 16;
  uint4 codes[kRowsPerWave];
  if (k < K)
    load_codes(k, codes);
  // (The first weights are in flight while the block forms the activation
  // codes of a folded norm.)
  uint8_t *codes_s = reinterpret_cast<uint8_t *>(chunk_s + kGemv8Rows * M * chunks);
  const bool folded = norm.x != nullptr;
  if (folded) {
    // The codes rms_norm would write, e4m3(bf16(norm(x)) * code_scale),
    // formed by this block into LDS.
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      const float *row = norm.x + m * norm.ld;
      const float denominator = row_norm_denominator(row, K, norm.eps, norm_partial);
      for (int c = tid * 4; c < K; c += 1024) {
        const float4 v = *reinterpret_cast<const float4 *>(row + c);
        const float4 g = *reinterpret_cast<const float4 *>(norm.scale + c);
        const float y[4] = {norm_value(v.x, denominator, g.x), norm_value(v.y, denominator, g.y),
                            norm_value(v.z, denominator, g.z), norm_value(v.w, denominator, g.w)};
        uint8_t code[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          code[e] = encode_e4m3(round_bf16(y[e]) * code_scale);
        *reinterpret_cast<uint32_t *>(codes_s + m * K + c) = __builtin_bit_cast(uint32_t, code);
      }
      __syncthreads();
    }
  }
  for (; k < K; k += 1024) {
    uint4 next[kRowsPerWave];
    if (k + 1024 < K)
      load_codes(k + 1024, next);
    float av[kM][16];
#pragma unroll
    for (int m = 0; m < kM; ++m)
      decode16(folded ? *reinterpret_cast<const uint4 *>(codes_s + m * K + k)
                      : *reinterpret_cast<const uint4 *>(a + static_cast<size_t>(m) * K + k),
               av[m]);
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
      float wv[16];
      decode16(codes[r], wv);
#pragma unroll
      for (int m = 0; m < kM; ++m) {
        float sum = 0.0F;
#pragma unroll
        for (int e = 0; e < 16; ++e)
          sum = fmaf(av[m][e], wv[e], sum);
#pragma unroll
        for (int offset = 1; offset < kLanesPerChunk; offset <<= 1)
          sum += __shfl_xor(sum, offset, 64);
        if ((lane % kLanesPerChunk) == 0)
          chunk_s[((wave * kRowsPerWave + r) * M + m) * chunks + k / kChunk] = sum;
      }
    }
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
      codes[r] = next[r];
  }
  __syncthreads();
  if (tid >= kGemv8Rows * kGemv8MaxM)
    return;
  const int r = tid / kGemv8MaxM, m = tid % kGemv8MaxM;
  const int row = blockIdx.x * kGemv8Rows + r;
  if (m >= M || row >= N)
    return;
  float acc = 0.0F;
  for (int c = 0; c < chunks; ++c)
    acc = truncate_e8m13(acc + chunk_s[(r * M + m) * chunks + c]);
  put(out, static_cast<size_t>(m) * N + row, round_bf16(acc * output_scale));
}

unsigned elementwise_grid(size_t n) {
  const size_t blocks = (n + 255) / 256;
  return static_cast<unsigned>(blocks < 16384 ? blocks : 16384);
}

}  // namespace

uint8_t e4m3_encode_host(float value) { return encode_e4m3(value); }

Status e4m3_quantize_f32(const float *x, size_t n, float scale, uint8_t *codes,
                         hipStream_t stream) {
  if (x == nullptr || codes == nullptr || n == 0 || !(scale > 0.0F) ||
      !__builtin_isfinite(scale))
    return {ErrorCode::kInvalidArgument, "e4m3_quantize: invalid arguments"};
  hipLaunchKernelGGL(quantize_f32_kernel, dim3(elementwise_grid(n)), dim3(256), 0,
                     stream, x, n, scale, codes);
  return launch_status("quantize_f32_kernel");
}

Status e4m3_quantize_bf16(const uint16_t *x, size_t n, float scale,
                          uint8_t *codes, hipStream_t stream) {
  if (x == nullptr || codes == nullptr || n == 0 || !(scale > 0.0F) ||
      !__builtin_isfinite(scale))
    return {ErrorCode::kInvalidArgument, "e4m3_quantize: invalid arguments"};
  hipLaunchKernelGGL(quantize_bf16_kernel, dim3(elementwise_grid(n)), dim3(256), 0,
                     stream, x, n, scale, codes);
  return launch_status("quantize_bf16_kernel");
}

template <typename Out>
Status fp8_linear_impl(const uint8_t *in_codes, const uint8_t *w_codes, Out *out,
                       size_t M, size_t N, size_t K, float output_scale,
                       Fp8Mode mode, hipStream_t stream, const RowNorm *norm = nullptr,
                       float code_scale = 0.0F) {
  if (norm != nullptr) {
    if (norm->x == nullptr || norm->scale == nullptr || M > static_cast<size_t>(kGemv8MaxM) ||
        K > static_cast<size_t>(kGemv8MaxK) || mode == kFp8Exact || K % kBK != 0 ||
        norm->ld < K || norm->ld % 4 != 0 || reinterpret_cast<uintptr_t>(norm->x) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(norm->scale) % 16 != 0 ||
        !(code_scale > 0.0F && __builtin_isfinite(code_scale)))
      return {ErrorCode::kInvalidArgument,
              "fp8_linear_normed: needs an MFMA mode, M <= 4, K <= 8192 (a multiple of 128), "
              "16-byte aligned F32 rows and scale, and a positive input scale"};
    in_codes = w_codes;  // not read
  }
  if (in_codes == nullptr || w_codes == nullptr || out == nullptr || M == 0 ||
      N == 0 || K == 0 || K % 32 != 0 || !(output_scale > 0.0F) ||
      !__builtin_isfinite(output_scale) || M > (1U << 30) || N > (1U << 30))
    return {ErrorCode::kInvalidArgument,
            "fp8_linear: invalid arguments (K must be a positive multiple of 32)"};
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  if (mode == kFp8Exact) {
    hipLaunchKernelGGL(qgmma_exact_kernel<Out>, dim3(ceil_div(N, kExactTile), ceil_div(M, kExactTile)),
                       dim3(256), 0, stream, in_codes, w_codes, out, m, n, k, output_scale);
    return launch_status("qgmma_exact_kernel");
  }
  if (K % kBK != 0)
    return {ErrorCode::kInvalidArgument, "fp8_linear: MFMA modes need K % 128 == 0"};
  if (mode != kFp8MfmaK32 && mode != kFp8MfmaK128)
    return {ErrorCode::kInvalidArgument, "fp8_linear: unknown mode"};
  if (M <= static_cast<size_t>(kGemv8MaxM) && K <= static_cast<size_t>(kGemv8MaxK)) {
    const dim3 grid(static_cast<unsigned>(ceil_div(N, kGemv8Rows)));
    const int chunk = mode == kFp8MfmaK32 ? 32 : 128;
    const size_t lds = kGemv8Rows * M * (K / chunk) * sizeof(float) +
                       (norm != nullptr ? M * K : 0);
    auto pick = [&](auto rows_c) {
      constexpr int kM = decltype(rows_c)::value;
      return mode == kFp8MfmaK32 ? fp8_gemv_kernel<32, kM, Out> : fp8_gemv_kernel<128, kM, Out>;
    };
    const auto kernel = M == 1   ? pick(std::integral_constant<int, 1>{})
                        : M == 2 ? pick(std::integral_constant<int, 2>{})
                        : M == 3 ? pick(std::integral_constant<int, 3>{})
                                 : pick(std::integral_constant<int, 4>{});
    if (lds > 64 * 1024)
      EVO_TRY(hip_status(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds)),
                         "fp8_gemv_kernel LDS opt-in"));
    const RowNorm folded = norm != nullptr ? *norm : RowNorm{nullptr, nullptr, 0.0F, 0};
    hipLaunchKernelGGL(kernel, grid, dim3(256), lds, stream, in_codes, w_codes, out, m, n, k,
                       output_scale, folded, code_scale);
    return launch_status("fp8_gemv_kernel");
  }
  const auto kernel = mode == kFp8MfmaK32 ? fp8_mfma_kernel<32, Out> : fp8_mfma_kernel<128, Out>;
  // 80 KB of the CU's 160 KB LDS (two blocks per CU): opt in above the
  // 64 KB default.
  EVO_TRY(hip_status(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(kMfmaLds)),
                     "fp8_mfma_kernel LDS opt-in"));
  const unsigned blocks = static_cast<unsigned>(ceil_div(M, kBM) * ceil_div(N, kBN));
  hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kWaves * 64), kMfmaLds, stream, in_codes, w_codes, out,
                     m, n, k, output_scale);
  return launch_status("fp8_mfma_kernel");
}

Status fp8_linear(const uint8_t *in_codes, const uint8_t *w_codes, float *out,
                  size_t M, size_t N, size_t K, float output_scale,
                  Fp8Mode mode, hipStream_t stream) {
  return fp8_linear_impl(in_codes, w_codes, out, M, N, K, output_scale, mode, stream);
}

Status fp8_linear(const uint8_t *in_codes, const uint8_t *w_codes, uint16_t *out,
                  size_t M, size_t N, size_t K, float output_scale,
                  Fp8Mode mode, hipStream_t stream) {
  return fp8_linear_impl(in_codes, w_codes, out, M, N, K, output_scale, mode, stream);
}

Status fp8_linear_normed(const RowNorm &norm, float input_scale, const uint8_t *w_codes,
                         uint16_t *out, size_t M, size_t N, size_t K, float output_scale,
                         Fp8Mode mode, hipStream_t stream) {
  return fp8_linear_impl(nullptr, w_codes, out, M, N, K, output_scale, mode, stream, &norm,
                         input_scale);
}

}  // namespace evo::hip
