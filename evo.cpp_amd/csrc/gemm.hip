// SPDX-License-Identifier: Apache-2.0
// Dense linears of the StripedHyena2 block on gfx950 MFMA.
//
//   C[M,N] = A[M,K] . W[N,K]^T  (+ fused epilogue)
//
// W is the BF16 weight in nn.Linear layout ([out, in], K contiguous); the
// accumulation is F32. Reference semantics: the F32-activation x BF16-weight
// dot of evo.cpp `src/cpu/model.cpp:284-314`.
//
// Activations arrive as split BF16 planes written by the producing kernel:
// hi = bf16(a) and lo = bf16(a - hi). With lo present ("split", profile
// hip-f32) both planes are multiplied by the exactly-BF16 weight, so each
// product carries ~16 significant bits of the activation (relative error
// ~2^-17) for twice the MFMA work; without lo (profile hip-bf16) one pass.
//
// Tiling for CDNA4: block tile 256 x 256, K step 32. The main kernel runs
// 512 threads = 8 waves as 4 (M) x 2 (N), each owning 64 x 128 = 4 x 8 MFMA
// 16x16x32 tiles (128 F32 accumulators per lane), two waves per SIMD so one
// wave's MFMAs cover the other's LDS reads and barrier waits. The short,
// wide wave tile reads 16 fragments per K step for 64 MFMAs in split mode
// (128 x 64 would read 20: A counts twice): 5-14 % faster on the 7B
// shapes. Operands reach
// LDS by DMA (global_load_lds_dwordx4) into XOR-swizzled, unpadded rows,
// triple-buffered. The fallback kernel (K % 32 != 0) runs 4 waves of
// 128 x 128 with register-staged, padded LDS rows.
// Tiles are renumbered so that each of the 8 XCDs (own L2) receives a
// contiguous band of the tile grid, walked in groups of 8 tile-rows.
#include <type_traits>

#include "common.hpp"
#include "row_norm.hpp"
#include "ops.hpp"

namespace evo::hip {
namespace {

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 32;
constexpr int kThreads = 256;
constexpr int kStride = kBK + 8;  // BF16 per LDS row

struct Epilogue {
  int mode;              // GemmEpilogue
  const uint16_t *bias;  // BF16 [N]
  const float *residual; // F32 [M, ldc]
  int gelu;              // gated: erf-GELU on the l1 half
  int gated_width;       // gated: valid output columns
};

__device__ inline float gelu_erf(const float x) {
  return 0.5F * x * (1.0F + erff(x * 0.7071067811865475244F));
}

template <bool kSplit>
__global__ __launch_bounds__(kThreads) void gemm_staged_kernel(
    const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int lda,
    const uint16_t *__restrict__ W, int M, int N, int K, float *__restrict__ C,
    uint16_t *__restrict__ c_hi, uint16_t *__restrict__ c_lo, int ldc,
    const Epilogue epi) {
  constexpr int kPlaneA = kBM * kStride;
  constexpr int kStage = (kSplit ? 2 : 1) * kPlaneA + kBN * kStride;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_m = wave >> 1;  // 0..1
  const int wave_n = wave & 1;   // 0..1
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, &tm, &tn);
  const int block_m = tm * kBM, block_n = tn * kBN;

  // Loader: each operand tile is 256 rows x 32 BF16 = 1024 x 16 B; thread t
  // moves chunks t + 256 v (v = 0..3): row = c / 4, 8-element segment c % 4.
  constexpr int kChunks = 1024 / kThreads;
  uint4 ra_hi[kChunks], ra_lo[kChunks], rw[kChunks];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int v = 0; v < kChunks; ++v) {
      const int c = tid + v * kThreads;
      const int r = c >> 2, k = k0 + (c & 3) * 8;
      const bool ka = k < K;
      const int ar = block_m + r, wr = block_n + r;
      const size_t a_off = static_cast<size_t>(ar) * lda + k;
      ra_hi[v] = (ar < M && ka) ? *reinterpret_cast<const uint4 *>(a_hi + a_off) : make_uint4(0, 0, 0, 0);
      if (kSplit)
        ra_lo[v] = (ar < M && ka) ? *reinterpret_cast<const uint4 *>(a_lo + a_off) : make_uint4(0, 0, 0, 0);
      rw[v] = (wr < N && ka) ? *reinterpret_cast<const uint4 *>(W + static_cast<size_t>(wr) * K + k)
                             : make_uint4(0, 0, 0, 0);
    }
  };
  auto stash = [&](int buffer) {
    uint16_t *stage = lds + buffer * kStage;
#pragma unroll
    for (int v = 0; v < kChunks; ++v) {
      const int c = tid + v * kThreads;
      const int r = c >> 2, seg = (c & 3) * 8;
      *reinterpret_cast<uint4 *>(stage + r * kStride + seg) = ra_hi[v];
      if (kSplit)
        *reinterpret_cast<uint4 *>(stage + kPlaneA + r * kStride + seg) = ra_lo[v];
      *reinterpret_cast<uint4 *>(stage + (kSplit ? 2 : 1) * kPlaneA + r * kStride + seg) = rw[v];
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[i][j][e] = 0.0F;

  const int steps = (K + kBK - 1) / kBK;
  fetch(0);
  stash(0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const int buffer = s & 1;
    if (s + 1 < steps)
      fetch((s + 1) * kBK);
    const uint16_t *stage = lds + buffer * kStage;
    const uint16_t *sa_hi = stage;
    const uint16_t *sa_lo = stage + kPlaneA;
    const uint16_t *sw = stage + (kSplit ? 2 : 1) * kPlaneA;
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      const int koff = ks + (lane >> 5) * 8;
      bf16x8 b[4], ah[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const bf16x8 *>(
            sw + (wave_n * 128 + j * 32 + (lane & 31)) * kStride + koff);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ah[i] = *reinterpret_cast<const bf16x8 *>(
            sa_hi + (wave_m * 128 + i * 32 + (lane & 31)) * kStride + koff);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], b[j], acc[i][j], 0, 0, 0);
      if (kSplit) {
        bf16x8 al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          al[i] = *reinterpret_cast<const bf16x8 *>(
              sa_lo + (wave_m * 128 + i * 32 + (lane & 31)) * kStride + koff);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
    if (s + 1 < steps)
      stash(buffer ^ 1);
    __syncthreads();
  }

  // Epilogue. Accumulator e of tile (i, j): row i*32 + (e/4)*8 + (lane/32)*4
  // + e%4 and column j*32 + lane%32 of the wave's 128 x 128 sub-tile.
  const int wave_col = block_n + wave_n * 128;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = block_m + wave_m * 128 + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
      if (row >= M)
        continue;
      if (epi.mode == kGemmGated) {
        // Columns [64q, 64q+32) hold l1 rows and [64q+32, 64q+64) the
        // matching l2 rows: tiles (0,1) and (2,3) pair up in-lane.
#pragma unroll
        for (int pair = 0; pair < 2; ++pair) {
          const int out_col = wave_col / 2 + pair * 32 + (lane & 31);
          if (out_col < epi.gated_width) {
            const float first = acc[i][2 * pair][e];
            const float value = (epi.gelu ? gelu_erf(first) : first) * acc[i][2 * pair + 1][e];
            const size_t index = static_cast<size_t>(row) * ldc + out_col;
            const uint16_t hi = f32_to_bf16(value);
            c_hi[index] = hi;
            if (c_lo != nullptr)
              c_lo[index] = f32_to_bf16(value - bf16_to_f32(hi));
          }
        }
        continue;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = wave_col + j * 32 + (lane & 31);
        if (col >= N)
          continue;
        float value = acc[i][j][e];
        const size_t index = static_cast<size_t>(row) * ldc + col;
        if (epi.mode == kGemmBias || epi.mode == kGemmBiasResidual)
          value = value + bf16_to_f32(epi.bias[col]);
        if (epi.mode == kGemmResidual || epi.mode == kGemmBiasResidual)
          value = value + epi.residual[index];
        C[index] = value;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Main kernel: operands move global -> LDS by DMA (global_load_lds_dwordx4),
// so no VGPRs stage them. LDS plane layout: 256 rows x four 16-byte units
// (32 BF16 of K); unit (row, seg) lives at row*4 + (seg ^ ((row >> 2) & 3)),
// which spreads the 16-byte fragment reads of 16 consecutive rows over all
// 64 banks without padding. One DMA instruction writes 64 consecutive units
// (16 rows), so lane l of instruction t loads row 16t + l/4, segment
// (l%4) ^ ((row >> 2) & 3). Three stages rotate: while step s is multiplied,
// steps s+1 and s+2 are in flight. Rows beyond M or N read a clamped valid
// row; their results are never stored. Requires K % 32 == 0.
constexpr int kStages = 3;
constexpr int kPlane = kBM * kBK;  // BF16 per plane (no padding)

__device__ inline int swizzled_unit(int row, int seg) {
  return row * 4 + (seg ^ ((row >> 2) & 3));
}

#ifndef EVO_GEMM_WAVES_M
#define EVO_GEMM_WAVES_M 4
#endif
// Wave layout of the 8 waves over the 256 x 256 block tile: kGemmWavesM (M)
// x 8 / kGemmWavesM (N). Per K step a wave reads (2 TM + TN) / 16 fragments
// (A has two planes in split mode) for 2 TM TN / 256 MFMAs, so the split
// product favours short, wide wave tiles: 64 x 128 reads 16 fragments per 64
// MFMAs, 128 x 64 reads 20.
constexpr int kGemmWavesM = EVO_GEMM_WAVES_M;
// Tile order: each XCD walks bands of 4 M tiles (tile_of), so its 32
// concurrent tiles form a 4 x 8 patch: 4 A panels (4 B per element, both
// planes) and 8 W panels in flight instead of 8 and 4 with bands of 8 --
// 20 % fewer L2 misses (FETCH_SIZE 1.81 -> 1.44 GB per MLP launch) at the
// same speed.
constexpr int kGemmGroupRows = 4;
constexpr int kGemmWavesN = 8 / kGemmWavesM;
constexpr int kGemmTM = kBM / kGemmWavesM, kGemmTN = kBN / kGemmWavesN;  // wave tile
constexpr int kGemmMI = kGemmTM / 16, kGemmNJ = kGemmTN / 16;            // 16 x 16 MFMA tiles
// CUs of the MI355X: one 256 x 256 tile per CU at a time (144 KB of LDS).
constexpr int kGemmCUs = 256;

// Epilogue of MFMA tile row i of a block tile (thread layout of
// gemm_kernel: 8 waves, wave (wave_m, wave_n) owns a kGemmTM x kGemmTN
// sub-tile). Accumulator e of tile (i, j): row i*16 + 4*(lane/16) + e,
// column j*16 + lane%16 of the sub-tile. Gated mode: columns [64q, 64q+32)
// hold l1 rows and [64q+32, 64q+64) the matching l2 rows, so tiles j and
// j+2 of each 64-column group pair up in-lane.
__device__ __attribute__((always_inline)) inline void gemm_epilogue_row(
    f32x4 (&acc)[kGemmNJ], int i, int block_m, int block_n, int wave_m, int wave_n, int lane,
    int M, int N, float *__restrict__ C, uint16_t *__restrict__ c_hi,
    uint16_t *__restrict__ c_lo, int ldc, const Epilogue &epi) {
  constexpr int kNJ = kGemmNJ;
  const int r16 = lane & 15;
  const int wave_col = block_n + wave_n * kGemmTN;
  const int wave_row = block_m + wave_m * kGemmTM + (lane >> 4) * 4;
  const bool bias_mode = epi.mode == kGemmBias || epi.mode == kGemmBiasResidual;
  const bool res_mode = epi.mode == kGemmResidual || epi.mode == kGemmBiasResidual;
  {
    if (epi.mode == kGemmGated) {
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        if ((j & 3) >= 2)
          continue;  // l2 tiles: consumed with their l1 partner
        const int col = wave_col / 2 + (j >> 2) * 32 + (j & 3) * 16 + r16;
        if (col >= epi.gated_width)
          continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = wave_row + i * 16 + e;
          if (row < M) {
            const float first = acc[j][e];
            const float value = (epi.gelu ? gelu_erf(first) : first) * acc[j + 2][e];
            const size_t index = static_cast<size_t>(row) * ldc + col;
            const uint16_t hi = f32_to_bf16(value);
            c_hi[index] = hi;
            if (c_lo != nullptr)
              c_lo[index] = f32_to_bf16(value - bf16_to_f32(hi));
          }
        }
      }
    } else {
      // Bias and residual for the whole row of tiles first, then the
      // stores: C may alias the residual, so a load placed after a store
      // would wait for it, one memory latency per value.
      if (bias_mode || res_mode) {
        float addend[kNJ][4];
#pragma unroll
        for (int j = 0; j < kNJ; ++j) {
          const int col = min(wave_col + j * 16 + r16, N - 1);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = min(wave_row + i * 16 + e, M - 1);
            addend[j][e] = res_mode ? epi.residual[static_cast<size_t>(row) * ldc + col] : 0.0F;
          }
        }
#pragma unroll
        for (int j = 0; j < kNJ; ++j) {
          const int col = min(wave_col + j * 16 + r16, N - 1);
          const float bias = bias_mode ? bf16_to_f32(epi.bias[col]) : 0.0F;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float value = acc[j][e];
            if (bias_mode)
              value = value + bias;
            if (res_mode)
              value = value + addend[j][e];
            acc[j][e] = value;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        const int col = wave_col + j * 16 + r16;
        if (col >= N)
          continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = wave_row + i * 16 + e;
          if (row < M)
            C[static_cast<size_t>(row) * ldc + col] = acc[j][e];
        }
      }
    }
  }
}

// Split K: block row blockIdx.y multiplies K range [y K, (y + 1) K) (K is
// the per-split length, ldw the weight row stride) into C + y c_split.
// Tail split: blocks [0, full_tiles) own whole tiles (the first full_tiles
// in tile order); each later pair of blocks takes one remaining tile, block
// 2t + h the K half h, and stores its raw accumulators in tail_part for
// gemm_tail_kernel. A launch whose last round would leave most CUs idle
// (352 tiles on 256 CUs) thus ends in a round of half-length tiles.
template <bool kSplit, bool kF16 = false>
__global__ __launch_bounds__(512) void gemm_kernel(
    const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int lda,
    const uint16_t *__restrict__ W, int ldw, int M, int N, int K, float *__restrict__ C,
    size_t c_split, uint16_t *__restrict__ c_hi, uint16_t *__restrict__ c_lo, int ldc,
    const Epilogue epi, int full_tiles, float *__restrict__ tail_part) {
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  int linear, half = -1;
  if (static_cast<int>(blockIdx.x) < full_tiles) {
    linear = xcd_linear(blockIdx.x, full_tiles);
  } else {
    const int t = blockIdx.x - full_tiles;
    linear = full_tiles + t / 2;
    half = t % 2;
  }
  int tm, tn;
  tile_of_linear<kGemmGroupRows>(linear, tiles_m, tiles_n, &tm, &tn);
  const int block_m = tm * kBM, block_n = tn * kBN;
  const int k_len = half < 0 ? K : K / 2;
  {
    const size_t k_first = static_cast<size_t>(blockIdx.y) * K + (half > 0 ? k_len : 0);
    a_hi += k_first;
    if (kSplit)
      a_lo += k_first;
    W += k_first;
    C += blockIdx.y * c_split;
  }
  constexpr int kWavesN = kGemmWavesN;
  constexpr int kTM = kGemmTM, kTN = kGemmTN;
  constexpr int kMI = kGemmMI, kNJ = kGemmNJ;
  constexpr int kPlanes = kSplit ? 3 : 2;  // A hi, (A lo), W
  constexpr int kStage = kPlanes * kPlane;
  // One-plane products stage 32 KB per K step: four stages (three steps of
  // DMA in flight) fit the LDS that three split stages take.
  constexpr int kSt = kSplit ? kStages : 4;
  __shared__ __attribute__((aligned(16))) uint16_t lds[kSt * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_m = wave / kWavesN;
  const int wave_n = wave % kWavesN;

  // This lane's DMA rows (instructions t = wave*2 + i) and segments.
  const uint16_t *src_a_hi[2], *src_a_lo[2], *src_w[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = wave * 2 + i;
    const int r = 16 * t + (lane >> 2);
    const int seg = (lane & 3) ^ ((r >> 2) & 3);
    const int ar = min(block_m + r, M - 1), wr = min(block_n + r, N - 1);
    src_a_hi[i] = a_hi + static_cast<size_t>(ar) * lda + seg * 8;
    src_a_lo[i] = kSplit ? a_lo + static_cast<size_t>(ar) * lda + seg * 8 : nullptr;
    src_w[i] = W + static_cast<size_t>(wr) * ldw + seg * 8;
  }
  // The A planes' DMAs go out before the weight's (issuing them
  // interleaved per row group measured 4 % slower on the MLP shape).
  auto issue = [&](int step) {
    uint16_t *stage = lds + (step % kSt) * kStage;
    const int k0 = step * kBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int unit0 = (wave * 2 + i) * 64;  // first unit of this instruction
      dma16(src_a_hi[i] + k0, stage + unit0 * 8);
      if (kSplit)
        dma16(src_a_lo[i] + k0, stage + kPlane + unit0 * 8);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
      dma16(src_w[i] + k0, stage + (kPlanes - 1) * kPlane + (wave * 2 + i) * 64 * 8);
  };

  f32x4 acc[kMI][kNJ];
#pragma unroll
  for (int i = 0; i < kMI; ++i)
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc[i][j][e] = 0.0F;

  const int steps = k_len / kBK;
  issue(0);
  if (steps > 1)
    issue(1);
  if (kSt > 3 && steps > 2)
    issue(2);
  const int seg = lane >> 4;
  const int r16 = lane & 15;
  for (int s = 0; s < steps; ++s) {
    // Wait for this wave's DMA of step s (the later steps' batches may stay
    // in flight: 6 DMAs per wave and step split, 4 one-plane), then for
    // every wave's.
    if constexpr (kSplit) {
      if (s + 1 < steps)
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
      if (s + 2 < steps)
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      else if (s + 1 < steps)
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    // The DMA of step s+kSt-1 (into the buffer of step s-1, which every
    // wave has left) is issued between the two MFMA halves, not here: the VMEM issue
    // then overlaps MFMAs instead of delaying the first fragment reads
    // (+2-6 %; raising the wave priority around the MFMAs measured neutral).
    const uint16_t *stage = lds + (s % kSt) * kStage;
    const uint16_t *sa_hi = stage;
    const uint16_t *sa_lo = stage + kPlane;
    const uint16_t *sw = stage + (kPlanes - 1) * kPlane;
    // One 16x16x32 fragment covers the whole K step: lane l reads row l%16
    // of its tile, 16-byte unit l/16. The fragments of the first half of
    // the longer dimension are read first; the reads of the second half
    // interleave with the MFMAs of the first (one LDS read, then a group of
    // MFMAs).
    // kF16: FP16 activation and weight (one pass, v_mfma_f32_16x16x32_f16).
    using Frag = std::conditional_t<kF16, f16x8, bf16x8>;
    Frag b[kNJ], ah[kMI], al[kMI];
    auto read_a = [&](int i) {
      ah[i] = *reinterpret_cast<const Frag *>(
          sa_hi + swizzled_unit(wave_m * kTM + i * 16 + r16, seg) * 8);
      if (kSplit)
        al[i] = *reinterpret_cast<const Frag *>(
            sa_lo + swizzled_unit(wave_m * kTM + i * 16 + r16, seg) * 8);
    };
    auto read_b = [&](int j) {
      b[j] = *reinterpret_cast<const Frag *>(
          sw + swizzled_unit(wave_n * kTN + j * 16 + r16, seg) * 8);
    };
    auto mfma = [&](int i, int j) {
      if constexpr (kF16) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b[j], acc[i][j], 0, 0, 0);
      } else {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], b[j], acc[i][j], 0, 0, 0);
        if (kSplit)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], b[j], acc[i][j], 0, 0, 0);
      }
    };
    if constexpr (kMI >= kNJ) {
      // tall wave tile: B whole, A in two halves
#pragma unroll
      for (int j = 0; j < kNJ; ++j)
        read_b(j);
#pragma unroll
      for (int i = 0; i < kMI / 2; ++i)
        read_a(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = kMI / 2; i < kMI; ++i)
        read_a(i);
#pragma unroll
      for (int i = 0; i < kMI / 2; ++i)
#pragma unroll
        for (int j = 0; j < kNJ; ++j)
          mfma(i, j);
      constexpr int kReads = (kMI / 2) * (kSplit ? 2 : 1);
      constexpr int kMfmas = (kMI / 2) * kNJ * (kSplit ? 2 : 1);
#pragma unroll
      for (int q = 0; q < kReads; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, kMfmas / kReads, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (s + kSt - 1 < steps)
        issue(s + kSt - 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = kMI / 2; i < kMI; ++i)
#pragma unroll
        for (int j = 0; j < kNJ; ++j)
          mfma(i, j);
    } else {
      // wide wave tile: A whole, B in two halves
#pragma unroll
      for (int i = 0; i < kMI; ++i)
        read_a(i);
#pragma unroll
      for (int j = 0; j < kNJ / 2; ++j)
        read_b(j);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = kNJ / 2; j < kNJ; ++j)
        read_b(j);
#pragma unroll
      for (int j = 0; j < kNJ / 2; ++j)
#pragma unroll
        for (int i = 0; i < kMI; ++i)
          mfma(i, j);
      constexpr int kReads = kNJ / 2;
      constexpr int kMfmas = kMI * (kNJ / 2) * (kSplit ? 2 : 1);
#pragma unroll
      for (int q = 0; q < kReads; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, kMfmas / kReads, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (s + kSt - 1 < steps)
        issue(s + kSt - 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = kNJ / 2; j < kNJ; ++j)
#pragma unroll
        for (int i = 0; i < kMI; ++i)
          mfma(i, j);
    }
  }

  if (half >= 0) {
    // Tail half: the raw accumulators, one coalesced 16-byte unit per lane
    // and MFMA tile; gemm_tail_kernel adds the halves and runs the epilogue.
    float *part = tail_part + static_cast<size_t>((linear - full_tiles) * 2 + half) * (kBM * kBN);
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int j = 0; j < kNJ; ++j)
        *reinterpret_cast<f32x4 *>(part + ((i * kNJ + j) * 512 + tid) * 4) = acc[i][j];
    return;
  }
#pragma unroll
  for (int i = 0; i < kMI; ++i)
    gemm_epilogue_row(acc[i], i, block_m, block_n, wave_m, wave_n, lane, M, N, C, c_hi, c_lo,
                      ldc, epi);
}

// Tail tiles of a gemm_kernel launch: the two K halves summed (first half
// first), then the tile's epilogue, in gemm_kernel's thread layout; block
// (t, i) takes MFMA tile row i of every wave of tail tile t, so that the
// reduction runs on kGemmMI blocks per tile.
__global__ __launch_bounds__(512) void gemm_tail_kernel(const float *__restrict__ tail_part,
                                                        int full_tiles, int M, int N,
                                                        float *__restrict__ C,
                                                        uint16_t *__restrict__ c_hi,
                                                        uint16_t *__restrict__ c_lo, int ldc,
                                                        const Epilogue epi) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_of_linear<kGemmGroupRows>(full_tiles + static_cast<int>(blockIdx.x), tiles_m, tiles_n,
                                 &tm, &tn);
  const float *first = tail_part + static_cast<size_t>(blockIdx.x) * 2 * (kBM * kBN);
  const float *second = first + kBM * kBN;
  const int i = blockIdx.y;
  f32x4 acc[kGemmNJ];
#pragma unroll
  for (int j = 0; j < kGemmNJ; ++j) {
    const int at = ((i * kGemmNJ + j) * 512 + tid) * 4;
    const f32x4 a = *reinterpret_cast<const f32x4 *>(first + at);
    const f32x4 b = *reinterpret_cast<const f32x4 *>(second + at);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[j][e] = a[e] + b[e];
  }
  gemm_epilogue_row(acc, i, tm * kBM, tn * kBN, wave / kGemmWavesN, wave % kGemmWavesN, lane, M,
                    N, C, c_hi, c_lo, ldc, epi);
}

// ---- Few-row product (decode, M <= 4): each 256-thread block owns 8
// weight rows and its 4 waves split K (wave w takes the 512-element K
// chunks w, w+4, ...); lane l reads K elements [k + 8 l, k + 8 l + 8) of a
// row, 1 KB coalesced per load. The activation row is hi + lo in F32 and
// the dot runs in F32 FMAs; wave partials are reduced by shuffles, then
// across the 4 waves through LDS. The weights are read once, so the
// product runs at the HBM rate the 256 x 256 tile kernel cannot reach with
// one row (it would fill N/256 CUs). Gated mode: the 8 rows are the l1 and
// l2 rows of 4 gated columns (32-row blocks alternate l1 / l2).
constexpr int kGemvRows = 8;
constexpr int kGemvMaxM = 4;

template <bool kSplit, int kM>
__global__ __launch_bounds__(256) void gemv_kernel(
    const uint16_t *__restrict__ a_hi, const uint16_t *__restrict__ a_lo, int lda,
    const uint16_t *__restrict__ W, int M, int N, int K, float *__restrict__ C,
    uint16_t *__restrict__ c_hi, uint16_t *__restrict__ c_lo, int ldc,
    const Epilogue epi, const RowNorm norm) {
  __shared__ float partial[4][kGemvRows][kGemvMaxM];
  __shared__ float norm_partial[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int unit = blockIdx.x;  // this block's 8 rows
  const bool gated = epi.mode == kGemmGated;
  int rows[kGemvRows];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) {
    if (gated) {
      const int column = unit * 4 + (r & 3);  // gated column
      rows[r] = (column / 32) * 64 + (r >= 4 ? 32 : 0) + column % 32;
    } else {
      rows[r] = unit * kGemvRows + r;
    }
  }
  float acc[kGemvRows][kM];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
    for (int m = 0; m < kM; ++m)
      acc[r][m] = 0.0F;
  // The weights of the wave's next K chunk are loaded before the current
  // chunk is multiplied, so two chunks (16 KB per wave) are in flight.
  auto load_w = [&](int k, uint4 (&wv)[kGemvRows]) {
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
      wv[r] = rows[r] < N ? *reinterpret_cast<const uint4 *>(
                                W + static_cast<size_t>(rows[r]) * K + k)
                          : make_uint4(0, 0, 0, 0);
  };
  int k = wave * 512 + lane * 8;
  uint4 wv[kGemvRows];
  if (k < K)
    load_w(k, wv);
  // Folded RMSNorm: the denominators of the block's activation rows, formed
  // while the first weights are in flight.
  float denominator[kM];
  if (norm.x != nullptr) {
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      denominator[m] = row_norm_denominator(norm.x + m * norm.ld, K, norm.eps, norm_partial);
      __syncthreads();
    }
  }
  for (; k < K; k += 2048) {
    uint4 wn[kGemvRows];
    if (k + 2048 < K)
      load_w(k + 2048, wn);
    float x[kM][8];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      if (norm.x != nullptr) {
        // The planes rms_norm would write: hi = bf16(y), lo = bf16(y - hi).
        const float *xs = norm.x + m * norm.ld + k;
        const float4 v0 = *reinterpret_cast<const float4 *>(xs);
        const float4 v1 = *reinterpret_cast<const float4 *>(xs + 4);
        const float4 g0 = *reinterpret_cast<const float4 *>(norm.scale + k);
        const float4 g1 = *reinterpret_cast<const float4 *>(norm.scale + k + 4);
        const float xv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float y = norm_value(xv[e], denominator[m], gv[e]);
          const float hi = bf16_to_f32(f32_to_bf16(y));
          x[m][e] = hi + (kSplit ? bf16_to_f32(f32_to_bf16(y - hi)) : 0.0F);
        }
        continue;
      }
      const uint4 h = *reinterpret_cast<const uint4 *>(a_hi + static_cast<size_t>(m) * lda + k);
      const uint16_t *hs = reinterpret_cast<const uint16_t *>(&h);
      uint4 l = make_uint4(0, 0, 0, 0);
      if (kSplit)
        l = *reinterpret_cast<const uint4 *>(a_lo + static_cast<size_t>(m) * lda + k);
      const uint16_t *ls = reinterpret_cast<const uint16_t *>(&l);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        x[m][e] = bf16_to_f32(hs[e]) + (kSplit ? bf16_to_f32(ls[e]) : 0.0F);
    }
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) {
      const uint16_t *ws = reinterpret_cast<const uint16_t *>(&wv[r]);
#pragma unroll
      for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          acc[r][m] = fmaf(x[m][e], bf16_to_f32(ws[e]), acc[r][m]);
    }
#pragma unroll
    for (int r = 0; r < kGemvRows; ++r)
      wv[r] = wn[r];
  }
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      float v = acc[r][m];
#pragma unroll
      for (int offset = 32; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset, 64);
      if (lane == 0)
        partial[wave][r][m] = v;
    }
  __syncthreads();
  if (wave != 0 || lane >= kM)
    return;
  const int m = lane;
  float total[kGemvRows];
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r)
    total[r] = partial[0][r][m] + partial[1][r][m] + partial[2][r][m] + partial[3][r][m];
  if (gated) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int column = unit * 4 + j;
      if (column >= epi.gated_width || rows[j + 4] >= N)
        continue;
      const float first = total[j], second = total[j + 4];
      const float value = (epi.gelu ? gelu_erf(first) : first) * second;
      const size_t index = static_cast<size_t>(m) * ldc + column;
      const uint16_t hi = f32_to_bf16(value);
      c_hi[index] = hi;
      if (c_lo != nullptr)
        c_lo[index] = f32_to_bf16(value - bf16_to_f32(hi));
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < kGemvRows; ++r) {
    const int column = rows[r];
    if (column >= N)
      continue;
    const size_t index = static_cast<size_t>(m) * ldc + column;
    float value = total[r];
    if (epi.mode == kGemmBias || epi.mode == kGemmBiasResidual)
      value = value + bf16_to_f32(epi.bias[column]);
    if (epi.mode == kGemmResidual || epi.mode == kGemmBiasResidual)
      value = value + epi.residual[index];
    C[index] = value;
  }
}

// Split BF16 planes (hi + lo) -> one FP16 plane of their sum (RNE,
// saturating), 8 elements per thread and step.
__global__ void planes_to_f16_kernel(const uint16_t *__restrict__ hi,
                                     const uint16_t *__restrict__ lo, size_t n8,
                                     _Float16 *__restrict__ out, int *saturated) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n8;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const uint4 h = reinterpret_cast<const uint4 *>(hi)[i];
    const uint4 l = reinterpret_cast<const uint4 *>(lo)[i];
    const uint32_t hw[4] = {h.x, h.y, h.z, h.w}, lw[4] = {l.x, l.y, l.z, l.w};
    f16x8 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float a = __builtin_bit_cast(float, hw[q] << 16) + __builtin_bit_cast(float, lw[q] << 16);
      const float b = __builtin_bit_cast(float, hw[q] & 0xffff0000U) +
                      __builtin_bit_cast(float, lw[q] & 0xffff0000U);
      note_f16_range(saturated, a);
      note_f16_range(saturated, b);
      v[2 * q] = static_cast<_Float16>(fminf(fmaxf(a, -65504.0F), 65504.0F));
      v[2 * q + 1] = static_cast<_Float16>(fminf(fmaxf(b, -65504.0F), 65504.0F));
    }
    reinterpret_cast<f16x8 *>(out)[i] = v;
  }
}

// BF16 -> FP16 (RNE, saturating), e.g. a weight for the FP16 product.
__global__ void bf16_to_f16_kernel(const uint16_t *__restrict__ x, size_t n,
                                   _Float16 *__restrict__ out) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = static_cast<_Float16>(fminf(fmaxf(bf16_to_f32(x[i]), -65504.0F), 65504.0F));
}

__global__ void split_kernel(const float *__restrict__ x, size_t n,
                             uint16_t *__restrict__ hi, uint16_t *__restrict__ lo) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const uint16_t h = f32_to_bf16(x[i]);
    hi[i] = h;
    if (lo != nullptr)
      lo[i] = f32_to_bf16(x[i] - bf16_to_f32(h));
  }
}

// Sum of the split-K partials in split order, then the epilogue:
// C[m, n] = sum_s part[s][m, n] (+ bias[n]) (+ residual[m, n]). Four columns
// per thread (N % 4 == 0); `vec`: C, the residual (16 bytes) and the bias
// (8 bytes) are aligned for vector accesses of the four (ldc % 4 == 0).
__global__ void split_k_reduce_kernel(const float *__restrict__ part, int splits, int M, int N,
                                      float *__restrict__ C, int ldc, const Epilogue epi,
                                      bool vec) {
  const size_t quads = static_cast<size_t>(M) * (N / 4);
  const size_t plane = static_cast<size_t>(M) * N;
  for (size_t q = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; q < quads;
       q += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t m = q / (N / 4);
    const int n = static_cast<int>(q % (N / 4)) * 4;
    f32x4 acc = *reinterpret_cast<const f32x4 *>(part + m * N + n);
    for (int sp = 1; sp < splits; ++sp) {
      const f32x4 v = *reinterpret_cast<const f32x4 *>(part + sp * plane + m * N + n);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc[e] = acc[e] + v[e];
    }
    const size_t index = m * ldc + n;
    const bool res_mode = epi.mode == kGemmResidual || epi.mode == kGemmBiasResidual;
    const bool bias_mode = epi.mode == kGemmBias || epi.mode == kGemmBiasResidual;
    // The residual loads ahead of the stores (C may alias the residual).
    float residual[4], bias[4];
    if (vec) {
      const f32x4 r = res_mode ? *reinterpret_cast<const f32x4 *>(epi.residual + index)
                               : f32x4{0.0F, 0.0F, 0.0F, 0.0F};
      const uint2 b = bias_mode ? *reinterpret_cast<const uint2 *>(epi.bias + n) : uint2{0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        residual[e] = r[e];
      bias[0] = __builtin_bit_cast(float, b.x << 16);
      bias[1] = __builtin_bit_cast(float, b.x & 0xffff0000U);
      bias[2] = __builtin_bit_cast(float, b.y << 16);
      bias[3] = __builtin_bit_cast(float, b.y & 0xffff0000U);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        residual[e] = res_mode ? epi.residual[index + e] : 0.0F;
        bias[e] = bias_mode ? bf16_to_f32(epi.bias[n + e]) : 0.0F;
      }
    }
    f32x4 value;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      value[e] = acc[e];
      if (bias_mode)
        value[e] = value[e] + bias[e];
      if (res_mode)
        value[e] = value[e] + residual[e];
    }
    if (vec) {
      *reinterpret_cast<f32x4 *>(C + index) = value;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        C[index + e] = value[e];
    }
  }
}

}  // namespace

Status planes_to_f16(const uint16_t *hi, const uint16_t *lo, size_t n, uint16_t *out,
                     hipStream_t stream, int *saturated) {
  if (hi == nullptr || lo == nullptr || out == nullptr || n % 8 != 0 ||
      reinterpret_cast<uintptr_t>(hi) % 16 != 0 || reinterpret_cast<uintptr_t>(lo) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(out) % 16 != 0)
    return {ErrorCode::kInvalidArgument,
            "planes_to_f16: 16-byte aligned planes of a multiple of 8 elements required"};
  const size_t n8 = n / 8;
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((n8 + 255) / 256, 16384));
  hipLaunchKernelGGL(planes_to_f16_kernel, dim3(blocks), dim3(256), 0, stream, hi, lo, n8,
                     reinterpret_cast<_Float16 *>(out), saturated);
  return launch_status("planes_to_f16_kernel");
}

Status bf16_to_f16(const uint16_t *x, size_t n, uint16_t *out, hipStream_t stream) {
  if (x == nullptr || out == nullptr)
    return {ErrorCode::kInvalidArgument, "bf16_to_f16: null buffer"};
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 16384));
  hipLaunchKernelGGL(bf16_to_f16_kernel, dim3(blocks), dim3(256), 0, stream, x, n,
                     reinterpret_cast<_Float16 *>(out));
  return launch_status("bf16_to_f16_kernel");
}

Status split_planes(const float *x, size_t n, uint16_t *hi, uint16_t *lo,
                    hipStream_t stream) {
  if (x == nullptr || hi == nullptr || n == 0)
    return {ErrorCode::kInvalidArgument, "split_planes: invalid arguments"};
  const unsigned grid = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 16384));
  hipLaunchKernelGGL(split_kernel, dim3(grid), dim3(256), 0, stream, x, n, hi, lo);
  return launch_status("split_kernel");
}

namespace {

// Shared body of gemm_bf16w (norm == nullptr) and gemm_bf16w_normed.
Status gemm_impl(const Activation &a, const RowNorm *norm, bool split, const uint16_t *W,
                 const GemmOutput &out, size_t M, size_t N, size_t K, GemmEpilogue mode,
                 const uint16_t *bias, const float *residual, bool gelu,
                 size_t gated_width, hipStream_t stream, float *split_workspace,
                 size_t split_workspace_bytes, SplitPartials *deferred) {
  if (deferred != nullptr)
    *deferred = SplitPartials{};
  if (norm != nullptr) {
    if (norm->x == nullptr || norm->scale == nullptr || M > static_cast<size_t>(kGemvMaxM) ||
        norm->ld < K || norm->ld % 4 != 0 ||
        reinterpret_cast<uintptr_t>(norm->x) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(norm->scale) % 16 != 0)
      return {ErrorCode::kInvalidArgument,
              "gemm_bf16w_normed: needs M <= 4 and 16-byte aligned F32 rows and scale"};
  } else if (a.hi == nullptr || a.ld < K || a.ld % 8 != 0) {
    return {ErrorCode::kInvalidArgument,
            "gemm_bf16w: null activation or unsupported stride (lda a multiple of 8)"};
  }
  if (W == nullptr || M == 0 || N == 0 || K == 0 || K % 8 != 0 ||
      M > (1U << 30) || N > (1U << 30) || K > (1U << 30))
    return {ErrorCode::kInvalidArgument,
            "gemm_bf16w: null operand or unsupported shape (K a multiple of 8)"};
  if ((mode == kGemmBias || mode == kGemmBiasResidual) && bias == nullptr)
    return {ErrorCode::kInvalidArgument, "gemm_bf16w: bias epilogue needs a bias"};
  if ((mode == kGemmResidual || mode == kGemmBiasResidual) && residual == nullptr)
    return {ErrorCode::kInvalidArgument, "gemm_bf16w: residual epilogue needs a residual"};
  if (mode == kGemmGated) {
    if (N % 64 != 0 || gated_width * 2 > N || out.hi == nullptr || out.ld < gated_width)
      return {ErrorCode::kInvalidArgument,
              "gemm_bf16w: gated epilogue needs N = 2*padded width (multiple of 64) "
              "and split-plane output"};
  } else if (out.f32 == nullptr || out.ld < N) {
    return {ErrorCode::kInvalidArgument, "gemm_bf16w: F32 output with ldc >= N required"};
  }
  if (a.f16 && (norm != nullptr || split || M <= static_cast<size_t>(kGemvMaxM) ||
                K % kBK != 0 || mode == kGemmGated))
    return {ErrorCode::kInvalidArgument,
            "gemm_bf16w: FP16 activations need one plane, more than 4 rows, K a multiple of 32 "
            "and a non-gated epilogue"};
  Epilogue epi{static_cast<int>(mode), bias, residual, gelu ? 1 : 0,
               static_cast<int>(gated_width)};
  const size_t tiles = static_cast<size_t>(ceil_div(M, kBM)) * ceil_div(N, kBN);
  if (tiles > (1U << 31))
    return {ErrorCode::kInvalidArgument, "gemm_bf16w: grid too large"};
  const dim3 grid(static_cast<unsigned>(tiles));
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  const int lda = static_cast<int>(a.ld), ldc = static_cast<int>(out.ld);
  if (M <= static_cast<size_t>(kGemvMaxM)) {
    const dim3 gemv_grid(static_cast<unsigned>(ceil_div(N, kGemvRows)));
    auto launch = [&](auto rows_c) {
      constexpr int kM = decltype(rows_c)::value;
      const RowNorm folded = norm != nullptr ? *norm : RowNorm{nullptr, nullptr, 0.0F, 0};
      if (split)
        hipLaunchKernelGGL((gemv_kernel<true, kM>), gemv_grid, dim3(256), 0, stream, a.hi,
                           a.lo, lda, W, m, n, k, out.f32, out.hi, out.lo, ldc, epi, folded);
      else
        hipLaunchKernelGGL((gemv_kernel<false, kM>), gemv_grid, dim3(256), 0, stream, a.hi,
                           a.lo, lda, W, m, n, k, out.f32, out.hi, out.lo, ldc, epi, folded);
    };
    switch (M) {
      case 1: launch(std::integral_constant<int, 1>{}); break;
      case 2: launch(std::integral_constant<int, 2>{}); break;
      case 3: launch(std::integral_constant<int, 3>{}); break;
      default: launch(std::integral_constant<int, 4>{}); break;
    }
    return launch_status("gemv_kernel");
  }
  if (K % kBK == 0) {
    // Few tiles (short prompts against W-wide outputs): split K so that about
    // one tile per CU runs, partials in the workspace, then one reduction.
    int splits = 1;
    // (The reduction reads the partials as 16-byte vectors.)
    if (mode != kGemmGated && split_workspace != nullptr &&
        reinterpret_cast<uintptr_t>(split_workspace) % 16 == 0 && N % 4 == 0 && tiles < 128) {
      for (int s = 2; s <= 16 && tiles * s <= 256; s *= 2)
        if (K % (static_cast<size_t>(s) * kBK) == 0 && K / s >= 8 * kBK &&
            static_cast<size_t>(s) * M * N * sizeof(float) <= split_workspace_bytes)
          splits = s;
    }
    if (splits > 1) {
      const Epilogue store{kGemmStore, nullptr, nullptr, 0, 0};
      const dim3 split_grid(static_cast<unsigned>(tiles), static_cast<unsigned>(splits));
      const int ks = k / splits;
      const size_t plane = M * N;
      const int all = static_cast<int>(tiles);
      if (split)
        hipLaunchKernelGGL(gemm_kernel<true>, split_grid, dim3(512), 0, stream, a.hi, a.lo,
                           lda, W, k, m, n, ks, split_workspace, plane, nullptr, nullptr, n,
                           store, all, nullptr);
      else if (a.f16)
        hipLaunchKernelGGL((gemm_kernel<false, true>), split_grid, dim3(512), 0, stream, a.hi,
                           a.lo, lda, W, k, m, n, ks, split_workspace, plane, nullptr, nullptr, n,
                           store, all, nullptr);
      else
        hipLaunchKernelGGL(gemm_kernel<false>, split_grid, dim3(512), 0, stream, a.hi, a.lo,
                           lda, W, k, m, n, ks, split_workspace, plane, nullptr, nullptr, n,
                           store, all, nullptr);
      EVO_TRY(launch_status("gemm_kernel (split K)"));
      if (deferred != nullptr && ldc == n) {
        const bool bias_mode = mode == kGemmBias || mode == kGemmBiasResidual;
        const bool res_mode = mode == kGemmResidual || mode == kGemmBiasResidual;
        *deferred = SplitPartials{split_workspace, splits, plane, bias_mode ? bias : nullptr,
                                  res_mode ? residual : nullptr};
        return Status::Ok();
      }
      const size_t quads = plane / 4;
      const unsigned blocks = static_cast<unsigned>(std::min<size_t>((quads + 255) / 256, 8192));
      const bool vec = ldc % 4 == 0 && reinterpret_cast<uintptr_t>(out.f32) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(residual) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(bias) % 8 == 0;
      hipLaunchKernelGGL(split_k_reduce_kernel, dim3(blocks), dim3(256), 0, stream,
                         split_workspace, splits, m, n, out.f32, ldc, epi, vec);
      return launch_status("split_k_reduce_kernel");
    }
    // Tail split: when the last round would hold at most half the CUs, its
    // tiles run as two K halves each (raw partials in the workspace), and
    // gemm_tail_kernel sums them in order and applies the epilogue.
    size_t tail = tiles > static_cast<size_t>(kGemmCUs) ? tiles % kGemmCUs : 0;
    if (tail == 0 || 2 * tail > static_cast<size_t>(kGemmCUs) || split_workspace == nullptr ||
        reinterpret_cast<uintptr_t>(split_workspace) % 16 != 0 || K % (2 * kBK) != 0 ||
        K / 2 < 8 * static_cast<size_t>(kBK) ||
        2 * tail * kBM * kBN * sizeof(float) > split_workspace_bytes)
      tail = 0;
    const int full = static_cast<int>(tiles - tail);
    const dim3 main_grid(static_cast<unsigned>(tiles + tail));
    if (split)
      hipLaunchKernelGGL(gemm_kernel<true>, main_grid, dim3(512), 0, stream, a.hi, a.lo, lda,
                         W, k, m, n, k, out.f32, size_t{0}, out.hi, out.lo, ldc, epi, full,
                         split_workspace);
    else if (a.f16)
      hipLaunchKernelGGL((gemm_kernel<false, true>), main_grid, dim3(512), 0, stream, a.hi, a.lo,
                         lda, W, k, m, n, k, out.f32, size_t{0}, out.hi, out.lo, ldc, epi, full,
                         split_workspace);
    else
      hipLaunchKernelGGL(gemm_kernel<false>, main_grid, dim3(512), 0, stream, a.hi, a.lo, lda,
                         W, k, m, n, k, out.f32, size_t{0}, out.hi, out.lo, ldc, epi, full,
                         split_workspace);
    if (tail == 0)
      return launch_status("gemm_kernel");
    EVO_TRY(launch_status("gemm_kernel (tail split)"));
    hipLaunchKernelGGL(gemm_tail_kernel, dim3(static_cast<unsigned>(tail), kGemmMI), dim3(512), 0,
                       stream,
                       split_workspace, full, m, n, out.f32, out.hi, out.lo, ldc, epi);
    return launch_status("gemm_tail_kernel");
  }
  if (split)
    hipLaunchKernelGGL(gemm_staged_kernel<true>, grid, dim3(kThreads), 0, stream, a.hi, a.lo,
                       lda, W, m, n, k, out.f32, out.hi, out.lo, ldc, epi);
  else
    hipLaunchKernelGGL(gemm_staged_kernel<false>, grid, dim3(kThreads), 0, stream, a.hi, a.lo,
                       lda, W, m, n, k, out.f32, out.hi, out.lo, ldc, epi);
  return launch_status("gemm_staged_kernel");
}

}  // namespace

Status gemm_bf16w(const Activation &a, const uint16_t *W, const GemmOutput &out,
                  size_t M, size_t N, size_t K, GemmEpilogue mode,
                  const uint16_t *bias, const float *residual, bool gelu,
                  size_t gated_width, hipStream_t stream, float *split_workspace,
                  size_t split_workspace_bytes, SplitPartials *deferred) {
  return gemm_impl(a, nullptr, a.lo != nullptr, W, out, M, N, K, mode, bias, residual, gelu,
                   gated_width, stream, split_workspace, split_workspace_bytes, deferred);
}

Status split_k_finish(const SplitPartials &src, float *C, size_t rows, size_t width,
                      hipStream_t stream) {
  if (src.splits == 0)
    return Status::Ok();
  if (src.part == nullptr || C == nullptr || width % 4 != 0 || src.plane != rows * width)
    return {ErrorCode::kInvalidArgument, "split_k_finish: invalid partials"};
  const GemmEpilogue mode = src.bias != nullptr
                                ? (src.residual != nullptr ? kGemmBiasResidual : kGemmBias)
                                : (src.residual != nullptr ? kGemmResidual : kGemmStore);
  const Epilogue epi{static_cast<int>(mode), src.bias, src.residual, 0, 0};
  const size_t quads = src.plane / 4;
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((quads + 255) / 256, 8192));
  const bool vec = reinterpret_cast<uintptr_t>(C) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(src.residual) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(src.bias) % 8 == 0;
  hipLaunchKernelGGL(split_k_reduce_kernel, dim3(blocks), dim3(256), 0, stream, src.part,
                     src.splits, static_cast<int>(rows), static_cast<int>(width), C,
                     static_cast<int>(width), epi, vec);
  return launch_status("split_k_reduce_kernel");
}

Status gemm_bf16w_normed(const RowNorm &norm, bool split, const uint16_t *W,
                         const GemmOutput &out, size_t M, size_t N, size_t K,
                         GemmEpilogue mode, const uint16_t *bias, const float *residual,
                         bool gelu, size_t gated_width, hipStream_t stream) {
  return gemm_impl(Activation{nullptr, nullptr, K}, &norm, split, W, out, M, N, K, mode, bias,
                   residual, gelu, gated_width, stream, nullptr, 0, nullptr);
}

}  // namespace evo::hip
