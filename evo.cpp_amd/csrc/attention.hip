// SPDX-License-Identifier: Apache-2.0
// Attention block of StripedHyena2 on gfx950 (prefill; single-query decode).
//
// qkv_rope: splits the Wqkv projection (head-major `column_split` layout
// [h][q,k,v][d], or component-major [q,k,v][h][d]), applies GPT-NeoX
// half-pair RoPE at position (prefix + row) / rope_scale and writes Q and the
// appended K rows as split BF16 planes (hi = bf16(x), lo = bf16(x - hi)).
// v_transpose appends V to the transposed value cache V^T [W][capacity]
// (row h*d_head + d), keys permuted inside every 16-key block by swapping
// bits 2 and 3 of the position, the order in which one MFMA lane holds the
// probabilities of a 16-key step (see below).
// Reference: evo.cpp `src/cpu/model.cpp:455-509`.
//
// causal_attention: softmax(q.k / sqrt(d)) v over keys [0, position].
// Reference semantics: `src/cpu/model.cpp:510-544` (full softmax; the online
// form below equals it up to F32 rounding).
//
// MFMA kernel (head_dim 32/64/128): one block = 8 waves x 32 queries of one
// head (two waves per SIMD share each K/V tile). K [64 keys][d] and V^T [d][64 keys] tiles of both
// planes are DMA'd (global_load_lds) into XOR-swizzled LDS, double buffered,
// so the next tile streams in while this one computes. Each wave computes
// S^T = K Q^T (keys x queries) with v_mfma_f32_32x32x16_bf16, so every lane
// owns one query: the running max and sum stay in-lane (plus one exchange
// with the lane holding the other half of the keys), and P^T is already in
// the B-operand layout of O^T += V^T P^T. Products use three BF16 passes
// (hi*hi + hi*lo + lo*hi), about 16 significant bits per operand, with F32
// accumulation; the exponential is exp2 of log2(e)-prescaled scores.
// head_dim 16 uses a VALU kernel (four lanes per query).
#include "common.hpp"
#include "ops.hpp"

namespace evo::hip {

// FP16-plane attention output without a per-value range check: the outputs
// are convex combinations of V rows, whose range qkv_rope checks as they
// enter the cache.
struct F16Plane {
  uint16_t *out;
};
__device__ inline void put(const F16Plane &o, size_t i, float v) {
  o.out[i] = f32_to_f16_sat(v);
}

namespace {

__device__ inline void put_split(uint16_t *hi, uint16_t *lo, size_t i, float v) {
  const uint16_t h = f32_to_bf16(v);
  hi[i] = h;
  lo[i] = f32_to_bf16(v - bf16_to_f32(h));
}

__device__ inline float get_split(const uint16_t *hi, const uint16_t *lo, size_t i) {
  return bf16_to_f32(hi[i]) + bf16_to_f32(lo[i]);
}

// Position of key `pos` inside the transposed value cache.
__host__ __device__ inline size_t vt_column(size_t pos) {
  return (pos & ~static_cast<size_t>(15)) | (pos & 3) | ((pos & 4) << 1) | ((pos & 8) >> 1);
}

__device__ inline size_t qkv_column(int column_split, size_t width, size_t head,
                                    size_t head_dim, size_t component, size_t dim) {
  return column_split ? head * 3 * head_dim + component * head_dim + dim
                      : component * width + head * head_dim + dim;
}

// One block per row; thread t owns rotation pair t % (head_dim / 2) of
// heads t / (head_dim / 2) + k * (512 / head_dim), so the pair's cosine and
// sine are evaluated once per row (head_dim / 2 divides 256 for head_dim 16
// to 128) and every wave reads and writes whole runs of consecutive dims.
__global__ __launch_bounds__(256) void qkv_rope_kernel(
    const float *__restrict__ projected, size_t width, size_t heads, int half,
    int column_split, const float *__restrict__ inv_freq, float rope_scale, size_t prefix,
    uint16_t *__restrict__ q, size_t q_plane, uint16_t *__restrict__ k_cache,
    size_t cache_plane) {
  const size_t row = blockIdx.x;
  const size_t head_dim = 2 * static_cast<size_t>(half);
  const int pair = static_cast<int>(threadIdx.x) % half;
  const int head_step = 256 / half;
  const float *src = projected + row * width * 3;
  const float position = static_cast<float>(prefix + row) / rope_scale;
  const float angle = position * inv_freq[pair];
  const float cosine = cosf(angle), sine = sinf(angle);
  for (size_t head = threadIdx.x / half; head < heads; head += head_step) {
    const size_t qi = row * width + head * head_dim;
    const size_t ki = (prefix + row) * width + head * head_dim;
    {
      const float first = src[qkv_column(column_split, width, head, head_dim, 0, pair)];
      const float second = src[qkv_column(column_split, width, head, head_dim, 0, half + pair)];
      put_split(q, q + q_plane, qi + pair, first * cosine - second * sine);
      put_split(q, q + q_plane, qi + half + pair, second * cosine + first * sine);
    }
    {
      const float first = src[qkv_column(column_split, width, head, head_dim, 1, pair)];
      const float second = src[qkv_column(column_split, width, head, head_dim, 1, half + pair)];
      put_split(k_cache, k_cache + cache_plane, ki + pair, first * cosine - second * sine);
      put_split(k_cache, k_cache + cache_plane, ki + half + pair, second * cosine + first * sine);
    }
  }
}

// V rows [rows, W] of the projection -> V^T planes at positions prefix..:
// a 64-position x 64-channel tile is read row-wise, transposed through LDS
// and written position-contiguous.
__global__ __launch_bounds__(256) void v_transpose_kernel(
    const float *__restrict__ projected, size_t rows, size_t width, size_t head_dim,
    int column_split, size_t prefix, uint16_t *__restrict__ vt_cache, size_t cache_plane,
    size_t capacity, int *range_flag) {
  __shared__ float tile[64][65];
  const int tid = threadIdx.x;
  const size_t r0 = blockIdx.x * 64ULL, c0 = blockIdx.y * 64ULL;
  const size_t channel = c0 + (tid & 63);
  bool out_of_range = false;
  for (int i = tid >> 6; i < 64; i += 4) {
    const size_t row = r0 + i;
    float value = 0.0F;
    if (row < rows && channel < width)
      value = projected[row * width * 3 +
                        qkv_column(column_split, width, channel / head_dim, head_dim, 2,
                                   channel % head_dim)];
    out_of_range |= !(__builtin_fabsf(value) <= 65504.0F);
    tile[tid & 63][i] = value;
  }
  if (range_flag != nullptr && out_of_range)
    atomicOr(range_flag, kFlagF16Range);
  __syncthreads();
  if (prefix % 16 == 0 && r0 + 64 <= rows && c0 + 64 <= width) {
    // Whole tile from a 16-aligned position: its 64 V^T columns per channel
    // are [prefix + r0, +64) in the permuted order; each lane packs 8 of
    // them (column j holds row vt_column(j), the permutation being its own
    // inverse) into one 16-byte store per plane.
    uint16_t *base = vt_cache + prefix + r0;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = tid + 256 * k, i = idx >> 3, unit = idx & 7;
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float a = tile[i][vt_column(8 * unit + e)];
        const float b = tile[i][vt_column(8 * unit + e + 1)];
        const uint16_t ha = f32_to_bf16(a), hb = f32_to_bf16(b);
        hi[e / 2] = ha | (static_cast<uint32_t>(hb) << 16);
        lo[e / 2] = f32_to_bf16(a - bf16_to_f32(ha)) |
                    (static_cast<uint32_t>(f32_to_bf16(b - bf16_to_f32(hb))) << 16);
      }
      const size_t at = (c0 + i) * capacity + 8 * unit;
      *reinterpret_cast<uint4 *>(base + at) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
      *reinterpret_cast<uint4 *>(base + cache_plane + at) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
    return;
  }
  for (int i = tid >> 6; i < 64; i += 4) {
    const size_t ch = c0 + i, row = r0 + (tid & 63);
    if (row < rows && ch < width)
      put_split(vt_cache, vt_cache + cache_plane, ch * capacity + vt_column(prefix + row),
                tile[i][tid & 63]);
  }
}

// ------------------------------------------------------------ MFMA kernel
constexpr int kQueriesPerWave = 32;
constexpr int kKeys = 64;
constexpr int kFlashWaves = 8;  // waves (query groups of 32) sharing a K/V tile

// Swizzle of a row of kUnits 16-byte units: 8 consecutive rows read at one
// logical unit hit 8 distinct 16-byte bank groups.
template <int kUnits>
__device__ inline int swizzle(int row, int unit) {
  return unit ^ ((row * kUnits / 16) & (kUnits - 1));
}

template <int kD, int kFlashWaves = kFlashWaves>
struct FlashShape {
  static constexpr int kKUnits = kD / 8;             // 16-byte units per K row
  static constexpr int kKPlane = kKeys * kD;         // BF16 per K plane
  static constexpr int kVPlane = kD * kKeys;         // BF16 per V^T plane
  static constexpr int kStage = 2 * kKPlane + 2 * kVPlane;
  static constexpr size_t kLdsBytes = 2 * kStage * sizeof(uint16_t);
  static constexpr int kChunksPerPlane = kD / 8;     // 1 KB chunks per K or V^T plane
  static constexpr int kDmaPerWave = 4 * kChunksPerPlane / kFlashWaves;
};

template <int kD, typename O, int kFlashWaves = kFlashWaves>
__global__ __launch_bounds__(kFlashWaves * 64) void flash_attention_kernel(
    const uint16_t *__restrict__ q, size_t q_plane, const uint16_t *__restrict__ k_cache,
    const uint16_t *__restrict__ vt_cache, size_t cache_plane, size_t capacity, size_t rows,
    size_t prefix, size_t heads, O out) {
  using Shape = FlashShape<kD, kFlashWaves>;
  constexpr int kDSteps = kD / 16;  // K-steps of S^T over head_dim
  constexpr int kDTiles = kD / 32;  // 32-row tiles of O^T
  extern __shared__ __attribute__((aligned(16))) uint16_t flash_lds[];

  const size_t width = heads * kD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, col = lane & 31;
  // Block -> (head, query block): heaviest (latest) query blocks first; with
  // heads % 8 == 0 the blocks of a head share an XCD (blocks are dealt to
  // the 8 XCDs round-robin), so its K/V tiles are reused from one L2.
  constexpr int kBlockQueries = kFlashWaves * kQueriesPerWave;
  const size_t query_blocks = (rows + kBlockQueries - 1) / kBlockQueries;
  const size_t b = blockIdx.x;
  size_t head, qb;
  if (heads % 8 == 0) {
    const size_t per_xcd = heads / 8, idx = b / 8;
    head = (b % 8) + 8 * (idx % per_xcd);
    qb = query_blocks - 1 - idx / per_xcd;
  } else {
    head = b % heads;
    qb = query_blocks - 1 - b / heads;
  }
  const size_t block_row = qb * kBlockQueries;
  const size_t row = block_row + wave * kQueriesPerWave + col;  // this lane's query
  const bool active = row < rows;
  const size_t position = prefix + row;
  // exp(x * scale) = exp2(x * scale * log2(e))
  const float scale2 = 1.4426950408889634F / sqrtf(static_cast<float>(kD));

  // Q^T operand fragments: for d-step s, 8 consecutive dims s*16 + half*8.
  bf16x8 qh[kDSteps], ql[kDSteps];
#pragma unroll
  for (int s = 0; s < kDSteps; ++s) {
    const size_t base = (active ? row : 0) * width + head * kD + s * 16 + half * 8;
    qh[s] = *reinterpret_cast<const bf16x8 *>(q + base);
    ql[s] = *reinterpret_cast<const bf16x8 *>(q + q_plane + base);
    if (!active) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qh[s][e] = static_cast<__bf16>(0.0F);
        ql[s][e] = static_cast<__bf16>(0.0F);
      }
    }
  }

  // Per-lane DMA sources of tile 0 (op g of this wave: part g / kChunksPerPlane
  // of {K hi, K lo, V hi, V lo}, 1 KB chunk g % kChunksPerPlane of that plane).
  const uint16_t *src[Shape::kDmaPerWave];
  int dst[Shape::kDmaPerWave];
#pragma unroll
  for (int i = 0; i < Shape::kDmaPerWave; ++i) {
    const int g = wave * Shape::kDmaPerWave + i;
    const int part = g / Shape::kChunksPerPlane, chunk = g % Shape::kChunksPerPlane;
    const int flat = chunk * 64 + lane;  // 16-byte unit within the plane
    if (part < 2) {
      const int key = flat / Shape::kKUnits, unit = swizzle<Shape::kKUnits>(key, flat % Shape::kKUnits);
      src[i] = k_cache + (part == 1 ? cache_plane : 0) + static_cast<size_t>(key) * width +
               head * kD + unit * 8;
      dst[i] = part * Shape::kKPlane + chunk * 512;
    } else {
      const int d = flat / 8, unit = swizzle<8>(d, flat % 8);
      src[i] = vt_cache + (part == 3 ? cache_plane : 0) +
               (head * kD + d) * capacity + unit * 8;
      dst[i] = 2 * Shape::kKPlane + (part - 2) * Shape::kVPlane + chunk * 512;
    }
  }
  auto issue = [&](size_t tile) {
    uint16_t *stage = flash_lds + (tile & 1) * Shape::kStage;
    const size_t k0 = tile * kKeys;
#pragma unroll
    for (int i = 0; i < Shape::kDmaPerWave; ++i) {
      const int g = wave * Shape::kDmaPerWave + i;
      const bool is_k = g / Shape::kChunksPerPlane < 2;
      dma16(src[i] + (is_k ? k0 * width : k0), stage + dst[i]);
    }
  };

  f32x16 o_acc[kDTiles];
#pragma unroll
  for (int t = 0; t < kDTiles; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      o_acc[t][e] = 0.0F;
  float running_max = -INFINITY, partial_sum = 0.0F;

  const size_t last_row = min(rows, block_row + kBlockQueries) - 1;
  const size_t tiles = (prefix + last_row + 1 + kKeys - 1) / kKeys;
  const size_t wave_first = prefix + block_row + wave * kQueriesPerWave;  // lowest position
  issue(0);
  for (size_t tile = 0; tile < tiles; ++tile) {
    // This wave's DMA of the tile (the only one in flight), then one
    // barrier: every wave's DMA of the tile has landed and every wave has
    // left buffer (tile+1)&1 (tile-1's), which the next DMA overwrites.
    wait_dma<0>();
    __syncthreads();
    if (tile + 1 < tiles)
      issue(tile + 1);
    const uint16_t *stage = flash_lds + (tile & 1) * Shape::kStage;
    const uint16_t *k_hi = stage, *k_lo = stage + Shape::kKPlane;
    const uint16_t *v_hi = stage + 2 * Shape::kKPlane, *v_lo = v_hi + Shape::kVPlane;
    const size_t k0 = tile * kKeys;

    // S^T tiles: st[kt] holds keys kt*32 + (e/4)*8 + half*4 + e%4 for query col.
    f32x16 st[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        st[kt][e] = 0.0F;
      const int key = kt * 32 + col;
#pragma unroll
      for (int s = 0; s < kDSteps; ++s) {
        const int off = (key * Shape::kKUnits + swizzle<Shape::kKUnits>(key, 2 * s + half)) * 8;
        const bf16x8 kh = *reinterpret_cast<const bf16x8 *>(k_hi + off);
        const bf16x8 kl = *reinterpret_cast<const bf16x8 *>(k_lo + off);
        st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qh[s], st[kt], 0, 0, 0);
        st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, ql[s], st[kt], 0, 0, 0);
        st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qh[s], st[kt], 0, 0, 0);
      }
    }
    // Scale (log2 domain), causal mask on the diagonal tiles, tile maximum.
    float tile_max = -INFINITY;
    const bool diagonal = k0 + kKeys - 1 > wave_first;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float value = st[kt][e] * scale2;
        if (diagonal) {
          const size_t key = k0 + kt * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
          value = key <= position ? value : -INFINITY;
        }
        st[kt][e] = value;
        tile_max = fmaxf(tile_max, value);
      }
    tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32, 64));
    const float new_max = fmaxf(running_max, tile_max);
    if (__any(new_max != running_max)) {
      // A query with no visible key yet keeps new_max = -inf: nothing to scale.
      const float correction =
          new_max == -INFINITY ? 1.0F : __builtin_amdgcn_exp2f(running_max - new_max);
      partial_sum *= correction;
#pragma unroll
      for (int t = 0; t < kDTiles; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          o_acc[t][e] *= correction;
      running_max = new_max;
    }
    const float base = new_max == -INFINITY ? 0.0F : new_max;
    // P = exp2(S - max) as B operands; with the permuted V^T key order, the
    // 8 entries e0..e0+7 of this lane are the 8 consecutive V^T columns of
    // 16-key step kk at half*8.
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int kt = kk >> 1, e0 = (kk & 1) * 8;
      bf16x8 ph, pl;
#pragma unroll
      for (int slot = 0; slot < 8; ++slot) {
        const float p = __builtin_amdgcn_exp2f(st[kt][e0 + slot] - base);
        partial_sum += p;
        const __bf16 h = static_cast<__bf16>(p);
        ph[slot] = h;
        pl[slot] = static_cast<__bf16>(p - static_cast<float>(h));
      }
#pragma unroll
      for (int t = 0; t < kDTiles; ++t) {
        const int d = t * 32 + col;
        const int off = (d * 8 + swizzle<8>(d, 2 * kk + half)) * 8;
        const bf16x8 vh = *reinterpret_cast<const bf16x8 *>(v_hi + off);
        const bf16x8 vl = *reinterpret_cast<const bf16x8 *>(v_lo + off);
        o_acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, ph, o_acc[t], 0, 0, 0);
        o_acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vh, pl, o_acc[t], 0, 0, 0);
        o_acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl, ph, o_acc[t], 0, 0, 0);
      }
    }
  }
  const float total = partial_sum + __shfl_xor(partial_sum, 32, 64);
  if (!active)
    return;
  // O^T entry e of tile t: d = t*32 + (e/4)*8 + half*4 + e%4, query = col.
#pragma unroll
  for (int t = 0; t < kDTiles; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int d = t * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
      put(out, row * width + head * kD + d, o_acc[t][e] / total);
    }
}

// ------------------------------------------------------------ VALU kernel
template <int kDim, typename O>  // head_dim, output type
__global__ __launch_bounds__(256) void attention_kernel(
    const uint16_t *__restrict__ q, size_t q_plane, const uint16_t *__restrict__ k_cache,
    const uint16_t *__restrict__ v_cache, size_t cache_plane, size_t capacity, size_t rows,
    size_t prefix, size_t heads, O out) {
  constexpr int kQ = 64, kTile = 64, kPart = kDim / 4;
  __shared__ float k_s[kTile * kDim];
  __shared__ float v_s[kTile * kDim];
  const size_t width = heads * kDim;
  const int tid = threadIdx.x;
  const int qi = tid >> 2, part = tid & 3;
  const size_t head = blockIdx.y;
  const size_t row = blockIdx.x * static_cast<size_t>(kQ) + qi;
  const bool active = row < rows;
  const size_t position = prefix + row;
  const float scale = 1.0F / sqrtf(static_cast<float>(kDim));
  float qv[kPart], acc[kPart];
#pragma unroll
  for (int d = 0; d < kPart; ++d) {
    qv[d] = active ? get_split(q, q + q_plane, row * width + head * kDim + part * kPart + d)
                   : 0.0F;
    acc[d] = 0.0F;
  }
  float running_max = -INFINITY, denominator = 0.0F;
  const size_t last_row = min(rows, blockIdx.x * static_cast<size_t>(kQ) + kQ) - 1;
  const size_t keys_needed = prefix + last_row + 1;
  for (size_t k0 = 0; k0 < keys_needed; k0 += kTile) {
    __syncthreads();
    for (int i = tid; i < kTile * kDim; i += 256) {
      const int key = i / kDim, d = i % kDim;
      const size_t g = (k0 + key) * width + head * kDim + d;
      const bool ok = k0 + key < keys_needed;
      k_s[i] = ok ? get_split(k_cache, k_cache + cache_plane, g) : 0.0F;
      v_s[i] = ok ? get_split(v_cache, v_cache + cache_plane,
                              (head * kDim + d) * capacity + vt_column(k0 + key))
                  : 0.0F;
    }
    __syncthreads();
    float scores[kTile];
    float tile_max = -INFINITY;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      float dot = 0.0F;
#pragma unroll
      for (int d = 0; d < kPart; ++d)
        dot += qv[d] * k_s[j * kDim + part * kPart + d];
      dot += __shfl_xor(dot, 1, 64);
      dot += __shfl_xor(dot, 2, 64);
      scores[j] = k0 + j <= position ? dot * scale : -INFINITY;
      tile_max = fmaxf(tile_max, scores[j]);
    }
    if (tile_max == -INFINITY)
      continue;  // every key of this tile lies beyond this query
    const float new_max = fmaxf(running_max, tile_max);
    const float correction = expf(running_max - new_max);
    denominator *= correction;
#pragma unroll
    for (int d = 0; d < kPart; ++d)
      acc[d] *= correction;
    running_max = new_max;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      const float p = expf(scores[j] - new_max);
      denominator += p;
#pragma unroll
      for (int d = 0; d < kPart; ++d)
        acc[d] += p * v_s[j * kDim + part * kPart + d];
    }
  }
  if (active) {
#pragma unroll
    for (int d = 0; d < kPart; ++d)
      put(out, row * width + head * kDim + part * kPart + d, acc[d] / denominator);
  }
}

template <int kD, typename O>
Status launch_flash(const uint16_t *q, size_t q_plane, const uint16_t *k_cache,
                    const uint16_t *v_cache, size_t cache_plane, size_t capacity, size_t rows,
                    size_t prefix, size_t heads, O out, hipStream_t stream) {
  constexpr size_t lds = FlashShape<kD>::kLdsBytes;
  static_assert(lds <= 160 * 1024, "LDS");
  // Blocks of 8 waves share each K/V tile among 256 queries; when that
  // leaves CUs idle (short chunks: 1024 rows x 32 heads = 128 blocks), blocks
  // of 4 waves (128 queries) fill twice as many.
  const bool half = ceil_div(rows, kFlashWaves * kQueriesPerWave) * heads < 256;
  const int waves = half ? kFlashWaves / 2 : kFlashWaves;
  auto kernel = half ? flash_attention_kernel<kD, O, kFlashWaves / 2>
                     : flash_attention_kernel<kD, O, kFlashWaves>;
  EVO_TRY(hip_status(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(lds)),
                     "flash_attention_kernel LDS opt-in"));
  const size_t blocks = ceil_div(rows, static_cast<size_t>(waves) * kQueriesPerWave) * heads;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(waves * 64), lds, stream,
                     q, q_plane, k_cache, v_cache, cache_plane, capacity, rows, prefix, heads,
                     out);
  return launch_status("flash_attention_kernel");
}


// ---- Single-query (decode) attention, split over the keys: one block per
// (head, chunk of 256 keys). Each lane scores one key (F32 dot of q with
// the key's hi + lo planes), the block takes its max and exponentials, and
// 256 threads form the chunk's P V with thread t on dimension t / 2 and
// keys of half t % 2 (reading the transposed value cache row of that
// dimension; its 16-key permutation swaps position bits 2 and 3, so column c
// holds key vt_column(c)). The chunk leaves (max, sum, o[d]); a second
// kernel per head rescales the chunks to the common max and sums them in
// chunk order. Full-softmax semantics as `src/cpu/model.cpp:510-544`.
constexpr int kDecodeKeys = 256;

template <int kD>
__global__ __launch_bounds__(256) void decode_attention_kernel(
    const uint16_t *__restrict__ q, size_t q_plane, const uint16_t *__restrict__ k_cache,
    const uint16_t *__restrict__ v_cache, size_t cache_plane, size_t capacity,
    size_t keys, size_t heads, float *__restrict__ part) {
  __shared__ float q_s[kD];
  __shared__ float p_s[kDecodeKeys];
  __shared__ float red_s[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t chunk = blockIdx.x, h = blockIdx.y;
  const size_t width = heads * kD;
  if (tid < kD)
    q_s[tid] = get_split(q, q + q_plane, h * kD + tid);
  __syncthreads();
  const size_t key = chunk * kDecodeKeys + tid;
  float score = -INFINITY;
  if (key < keys) {
    const uint16_t *k_hi = k_cache + key * width + h * kD;
    const uint16_t *k_lo = k_hi + cache_plane;
    float dot = 0.0F;
#pragma unroll
    for (int d0 = 0; d0 < kD; d0 += 8) {
      const uint4 hv = *reinterpret_cast<const uint4 *>(k_hi + d0);
      const uint4 lv = *reinterpret_cast<const uint4 *>(k_lo + d0);
      const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w}, lw[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float k0 = __builtin_bit_cast(float, hw[i] << 16) +
                         __builtin_bit_cast(float, lw[i] << 16);
        const float k1 = __builtin_bit_cast(float, hw[i] & 0xffff0000U) +
                         __builtin_bit_cast(float, lw[i] & 0xffff0000U);
        dot = fmaf(q_s[d0 + 2 * i], k0, dot);
        dot = fmaf(q_s[d0 + 2 * i + 1], k1, dot);
      }
    }
    score = dot * (1.0F / sqrtf(static_cast<float>(kD)));
  }
  float m = score;
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1)
    m = fmaxf(m, __shfl_xor(m, offset, 64));
  if (lane == 0)
    red_s[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red_s[0], red_s[1]), fmaxf(red_s[2], red_s[3]));
  const float p = key < keys ? expf(score - m) : 0.0F;
  p_s[tid] = p;
  float l = p;
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1)
    l += __shfl_xor(l, offset, 64);
  __syncthreads();  // p_s complete; red_s reads done
  if (lane == 0)
    red_s[wave] = l;
  // P V: thread t -> dimension t / 2 (t < 2 kD), keys of half t % 2.
  float o = 0.0F;
  const int d = tid >> 1, part_half = tid & 1;
  if (d < kD) {
    const size_t row = h * kD + d;
    const size_t col0 = chunk * kDecodeKeys + part_half * (kDecodeKeys / 2);
    const uint16_t *v_hi = v_cache + row * capacity + col0;
    const uint16_t *v_lo = v_hi + cache_plane;
    // Whole 16-column blocks: the permutation moves a key up to 8 columns
    // past its position inside its block (key 84 of 85 sits in column 88).
    const size_t end = min(static_cast<size_t>(kDecodeKeys / 2),
                           keys > col0 ? (keys - col0 + 15) / 16 * 16 : size_t{0});
    for (size_t c0 = 0; c0 < end; c0 += 8) {
      const uint4 hv = *reinterpret_cast<const uint4 *>(v_hi + c0);
      const uint4 lv = *reinterpret_cast<const uint4 *>(v_lo + c0);
      const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w}, lw[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const size_t c = part_half * (kDecodeKeys / 2) + c0 + 2 * i;
        const float v0 = __builtin_bit_cast(float, hw[i] << 16) +
                         __builtin_bit_cast(float, lw[i] << 16);
        const float v1 = __builtin_bit_cast(float, hw[i] & 0xffff0000U) +
                         __builtin_bit_cast(float, lw[i] & 0xffff0000U);
        // Zero weights are skipped: columns of keys past the end may hold
        // unwritten cache.
        const float p0 = p_s[vt_column(c)], p1 = p_s[vt_column(c + 1)];
        if (p0 != 0.0F)
          o = fmaf(p0, v0, o);
        if (p1 != 0.0F)
          o = fmaf(p1, v1, o);
      }
    }
  }
  o += __shfl_xor(o, 1, 64);
  __syncthreads();
  float *dst = part + (h * gridDim.x + chunk) * (kD + 2);
  if (d < kD && part_half == 0)
    dst[2 + d] = o;
  if (tid == 0) {
    dst[0] = m;
    dst[1] = red_s[0] + red_s[1] + red_s[2] + red_s[3];
  }
}

template <int kD, typename O>
__global__ void decode_combine_kernel(const float *__restrict__ part, int chunks, O out) {
  const size_t h = blockIdx.x;
  const int d = threadIdx.x;
  const float *base = part + h * chunks * (kD + 2);
  float m = -INFINITY;
  for (int c = 0; c < chunks; ++c)
    m = fmaxf(m, base[c * (kD + 2)]);
  float l = 0.0F, o = 0.0F;
  for (int c = 0; c < chunks; ++c) {
    const float scale = expf(base[c * (kD + 2)] - m);
    l = fmaf(base[c * (kD + 2) + 1], scale, l);
    o = fmaf(base[c * (kD + 2) + 2 + d], scale, o);
  }
  put(out, h * kD + d, o / l);
}

template <int kD, typename O>
Status launch_decode(const uint16_t *q, size_t q_plane, const uint16_t *k_cache,
                     const uint16_t *v_cache, size_t cache_plane, size_t capacity, size_t keys,
                     size_t heads, float *workspace, O out, hipStream_t stream) {
  const unsigned chunks = static_cast<unsigned>(ceil_div(keys, kDecodeKeys));
  hipLaunchKernelGGL(decode_attention_kernel<kD>, dim3(chunks, heads), dim3(256), 0, stream, q,
                     q_plane, k_cache, v_cache, cache_plane, capacity, keys, heads, workspace);
  EVO_TRY(launch_status("decode_attention_kernel"));
  hipLaunchKernelGGL((decode_combine_kernel<kD, O>), dim3(heads), dim3(kD), 0, stream,
                     workspace, static_cast<int>(chunks), out);
  return launch_status("decode_combine_kernel");
}

template <typename O>
Status launch_attention(const uint16_t *q, size_t q_plane, const uint16_t *k_cache,
                        const uint16_t *v_cache, size_t cache_plane, size_t capacity,
                        size_t rows, size_t prefix, size_t heads, size_t head_dim, O out,
                        hipStream_t stream) {
  switch (head_dim) {
  case 16:
    hipLaunchKernelGGL((attention_kernel<16, O>), dim3(ceil_div(rows, 64), heads), dim3(256),
                       0, stream, q, q_plane, k_cache, v_cache, cache_plane, capacity, rows,
                       prefix, heads, out);
    return launch_status("attention_kernel");
  case 32:
    return launch_flash<32, O>(q, q_plane, k_cache, v_cache, cache_plane, capacity, rows,
                               prefix, heads, out, stream);
  case 64:
    return launch_flash<64, O>(q, q_plane, k_cache, v_cache, cache_plane, capacity, rows,
                               prefix, heads, out, stream);
  case 128:
    return launch_flash<128, O>(q, q_plane, k_cache, v_cache, cache_plane, capacity, rows,
                                prefix, heads, out, stream);
  default:
    return {ErrorCode::kUnsupported,
            "causal_attention: head_dim must be 16, 32, 64 or 128"};
  }
}

}  // namespace

Status qkv_rope(const float *projected, size_t rows, size_t width, size_t heads,
                bool column_split, const float *inv_freq, float rope_scale,
                size_t prefix, uint16_t *q, size_t q_plane, uint16_t *k_cache,
                uint16_t *v_cache, size_t cache_plane, size_t capacity, hipStream_t stream,
                int *v_range_flag) {
  if (projected == nullptr || inv_freq == nullptr || q == nullptr ||
      k_cache == nullptr || v_cache == nullptr || rows == 0 || heads == 0 ||
      width % heads != 0 || (width / heads) % 2 != 0 || !(rope_scale > 0.0F) ||
      q_plane < rows * width || capacity % kKeys != 0 || prefix + rows > capacity ||
      cache_plane < capacity * width)
    return {ErrorCode::kInvalidArgument, "qkv_rope: invalid arguments"};
  const size_t half = width / heads / 2;
  if (256 % half != 0 || rows > (1U << 31))
    return {ErrorCode::kInvalidArgument, "qkv_rope: head_dim / 2 must divide 256"};
  hipLaunchKernelGGL(qkv_rope_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream,
                     projected, width, heads, static_cast<int>(half), column_split ? 1 : 0,
                     inv_freq, rope_scale, prefix, q, q_plane, k_cache, cache_plane);
  EVO_TRY(launch_status("qkv_rope_kernel"));
  hipLaunchKernelGGL(v_transpose_kernel, dim3(ceil_div(rows, 64), ceil_div(width, 64)),
                     dim3(256), 0, stream, projected, rows, width, width / heads,
                     column_split ? 1 : 0, prefix, v_cache, cache_plane, capacity,
                     v_range_flag);
  return launch_status("v_transpose_kernel");
}

Status causal_attention(const uint16_t *q, size_t q_plane, const uint16_t *k_cache,
                        const uint16_t *v_cache, size_t cache_plane, size_t capacity,
                        size_t rows, size_t prefix, size_t heads, size_t head_dim,
                        float *out_f32, uint16_t *out_hi, uint16_t *out_lo,
                        hipStream_t stream, float *workspace, size_t workspace_bytes,
                        bool out_f16) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      (out_f32 == nullptr && out_hi == nullptr) || rows == 0 || heads == 0 ||
      heads > 65535 || q_plane < rows * heads * head_dim || capacity % kKeys != 0 ||
      prefix + rows > capacity || cache_plane < capacity * heads * head_dim)
    return {ErrorCode::kInvalidArgument, "causal_attention: invalid arguments"};
  // One query with a workspace for the chunk partials: split over the keys.
  const size_t keys = prefix + 1;
  if (rows == 1 && workspace != nullptr &&
      (head_dim == 32 || head_dim == 64 || head_dim == 128) &&
      heads * ceil_div(keys, kDecodeKeys) * (head_dim + 2) * sizeof(float) <= workspace_bytes) {
    auto run = [&](auto out) -> Status {
      switch (head_dim) {
      case 32:
        return launch_decode<32>(q, q_plane, k_cache, v_cache, cache_plane, capacity, keys,
                                 heads, workspace, out, stream);
      case 64:
        return launch_decode<64>(q, q_plane, k_cache, v_cache, cache_plane, capacity, keys,
                                 heads, workspace, out, stream);
      default:
        return launch_decode<128>(q, q_plane, k_cache, v_cache, cache_plane, capacity, keys,
                                  heads, workspace, out, stream);
      }
    };
    if (out_f32 != nullptr)
      return run(out_f32);
    if (out_f16)
      return run(F16Plane{out_hi});
    return run(SplitOut{out_hi, out_lo});
  }
  if (out_f32 != nullptr)
    return launch_attention(q, q_plane, k_cache, v_cache, cache_plane, capacity, rows, prefix,
                            heads, head_dim, out_f32, stream);
  if (out_f16)
    return launch_attention(q, q_plane, k_cache, v_cache, cache_plane, capacity, rows, prefix,
                            heads, head_dim, F16Plane{out_hi}, stream);
  return launch_attention(q, q_plane, k_cache, v_cache, cache_plane, capacity, rows, prefix,
                          heads, head_dim, SplitOut{out_hi, out_lo}, stream);
}

}  // namespace evo::hip
