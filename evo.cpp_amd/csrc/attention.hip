// SPDX-License-Identifier: Apache-2.0
// Attention block of StripedHyena2 on gfx950 (prefill).
//
// qkv_rope: splits the Wqkv projection (head-major `column_split` layout
// [h][q,k,v][d], or component-major [q,k,v][h][d]), applies GPT-NeoX
// half-pair RoPE at position (prefix + row) / rope_scale and writes Q and the
// appended K/V rows as split BF16 planes (hi = bf16(x), lo = bf16(x - hi)).
// Reference: evo.cpp `src/cpu/model.cpp:455-509`.
//
// causal_attention: softmax(q.k / sqrt(d)) v over keys [0, position].
// Reference semantics: `src/cpu/model.cpp:510-544` (full softmax; the online
// form below equals it up to F32 rounding).
//
// MFMA kernel (head_dim 32/64/128): one 256-thread block = 4 waves x 32
// queries of one head; K and V^T tiles of 64 keys are staged in LDS as BF16
// planes. Each wave computes S^T = K Q^T (keys x queries) with
// v_mfma_f32_32x32x16_bf16, so every lane owns one query: the running max
// and sum stay in-lane (plus one exchange with the lane holding the other
// half of the keys), and P^T is already in the B-operand layout of
// O^T += V^T P^T. Products use three BF16 passes (hi*hi + hi*lo + lo*hi),
// about 16 significant bits per operand, with F32 accumulation.
// head_dim 16 uses a VALU kernel (four lanes per query).
#include "common.hpp"
#include "ops.hpp"

namespace evo::hip {
namespace {

__device__ inline void put_split(uint16_t *hi, uint16_t *lo, size_t i, float v) {
  const uint16_t h = f32_to_bf16(v);
  hi[i] = h;
  lo[i] = f32_to_bf16(v - bf16_to_f32(h));
}

__device__ inline float get_split(const uint16_t *hi, const uint16_t *lo, size_t i) {
  return bf16_to_f32(hi[i]) + bf16_to_f32(lo[i]);
}

__global__ void qkv_rope_kernel(const float *__restrict__ projected, size_t rows,
                                size_t width, size_t heads, size_t head_dim,
                                int column_split, const float *__restrict__ inv_freq,
                                float rope_scale, size_t prefix, uint16_t *__restrict__ q,
                                size_t q_plane, uint16_t *__restrict__ k_cache,
                                uint16_t *__restrict__ v_cache, size_t cache_plane) {
  const size_t half = head_dim / 2;
  const size_t n = rows * heads * half;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
       i < n; i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t pair = i % half;
    const size_t head = (i / half) % heads;
    const size_t row = i / (half * heads);
    const float *src = projected + row * width * 3;
    auto source = [&](size_t component, size_t dim) {
      return column_split ? head * 3 * head_dim + component * head_dim + dim
                          : component * width + head * head_dim + dim;
    };
    const float position = static_cast<float>(prefix + row) / rope_scale;
    const float angle = position * inv_freq[pair];
    const float cosine = cosf(angle), sine = sinf(angle);
    const size_t qi = row * width + head * head_dim;
    const size_t ki = (prefix + row) * width + head * head_dim;
    {
      const float first = src[source(0, pair)], second = src[source(0, half + pair)];
      put_split(q, q + q_plane, qi + pair, first * cosine - second * sine);
      put_split(q, q + q_plane, qi + half + pair, second * cosine + first * sine);
    }
    {
      const float first = src[source(1, pair)], second = src[source(1, half + pair)];
      put_split(k_cache, k_cache + cache_plane, ki + pair, first * cosine - second * sine);
      put_split(k_cache, k_cache + cache_plane, ki + half + pair, second * cosine + first * sine);
    }
    put_split(v_cache, v_cache + cache_plane, ki + pair, src[source(2, pair)]);
    put_split(v_cache, v_cache + cache_plane, ki + half + pair, src[source(2, half + pair)]);
  }
}

// ------------------------------------------------------------ MFMA kernel
constexpr int kQueriesPerWave = 32;
constexpr int kKeys = 64;

template <int kD, typename O>
__global__ __launch_bounds__(256) void flash_attention_kernel(
    const uint16_t *__restrict__ q, size_t q_plane, const uint16_t *__restrict__ k_cache,
    const uint16_t *__restrict__ v_cache, size_t cache_plane, size_t rows, size_t prefix,
    size_t heads, O out) {
  constexpr int kKStride = kD + 8;     // K tile row (BF16), padded
  constexpr int kVStride = kKeys + 8;  // V^T tile row (BF16), padded
  constexpr int kDSteps = kD / 16;     // K-steps of S^T over head_dim
  constexpr int kDTiles = kD / 32;     // 32-row tiles of O^T
  __shared__ __attribute__((aligned(16))) uint16_t k_s[2][kKeys * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t v_s[2][kD * kVStride];

  const size_t width = heads * kD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, col = lane & 31;
  const size_t head = blockIdx.y;
  const size_t block_row = blockIdx.x * static_cast<size_t>(4 * kQueriesPerWave);
  const size_t row = block_row + wave * kQueriesPerWave + col;  // this lane's query
  const bool active = row < rows;
  const size_t position = prefix + row;
  const float scale = 1.0F / sqrtf(static_cast<float>(kD));

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
  f32x16 o_acc[kDTiles];
#pragma unroll
  for (int t = 0; t < kDTiles; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      o_acc[t][e] = 0.0F;
  float running_max = -INFINITY, partial_sum = 0.0F;

  const size_t last_row = min(rows, block_row + 4 * kQueriesPerWave) - 1;
  const size_t keys_needed = prefix + last_row + 1;
  for (size_t k0 = 0; k0 < keys_needed; k0 += kKeys) {
    __syncthreads();
    // K tile [key][d] and V^T tile [d][key], both planes.
    for (int c = tid; c < kKeys * kD / 8; c += 256) {
      const int key = c / (kD / 8), d0 = (c % (kD / 8)) * 8;
      const size_t g = (k0 + key) * width + head * kD + d0;
      uint4 kh = make_uint4(0, 0, 0, 0), kl = kh, vh = kh, vl = kh;
      if (k0 + key < keys_needed) {
        kh = *reinterpret_cast<const uint4 *>(k_cache + g);
        kl = *reinterpret_cast<const uint4 *>(k_cache + cache_plane + g);
        vh = *reinterpret_cast<const uint4 *>(v_cache + g);
        vl = *reinterpret_cast<const uint4 *>(v_cache + cache_plane + g);
      }
      *reinterpret_cast<uint4 *>(&k_s[0][key * kKStride + d0]) = kh;
      *reinterpret_cast<uint4 *>(&k_s[1][key * kKStride + d0]) = kl;
      const uint16_t *vhs = reinterpret_cast<const uint16_t *>(&vh);
      const uint16_t *vls = reinterpret_cast<const uint16_t *>(&vl);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v_s[0][(d0 + e) * kVStride + key] = vhs[e];
        v_s[1][(d0 + e) * kVStride + key] = vls[e];
      }
    }
    __syncthreads();

    // S^T tiles: st[kt] holds keys kt*32 + (e/4)*8 + half*4 + e%4 for query col.
    f32x16 st[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        st[kt][e] = 0.0F;
#pragma unroll
      for (int s = 0; s < kDSteps; ++s) {
        const int off = (kt * 32 + col) * kKStride + s * 16 + half * 8;
        const bf16x8 kh = *reinterpret_cast<const bf16x8 *>(&k_s[0][off]);
        const bf16x8 kl = *reinterpret_cast<const bf16x8 *>(&k_s[1][off]);
        st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qh[s], st[kt], 0, 0, 0);
        st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, ql[s], st[kt], 0, 0, 0);
        st[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qh[s], st[kt], 0, 0, 0);
      }
    }
    // Scale, causal mask, tile maximum.
    float tile_max = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const size_t key = k0 + kt * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
        const float value = key <= position ? st[kt][e] * scale : -INFINITY;
        st[kt][e] = value;
        tile_max = fmaxf(tile_max, value);
      }
    tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32, 64));
    const float new_max = fmaxf(running_max, tile_max);
    // A query with no visible key yet keeps new_max = -inf: nothing to scale.
    const float correction = new_max == -INFINITY ? 1.0F : expf(running_max - new_max);
    running_max = new_max;
    partial_sum *= correction;
#pragma unroll
    for (int t = 0; t < kDTiles; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        o_acc[t][e] *= correction;
    // P = exp(S - max) as B operands (P^T slots = this lane's key entries).
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int kt = kk >> 1, e0 = (kk & 1) * 8;
      bf16x8 ph, pl;
#pragma unroll
      for (int slot = 0; slot < 8; ++slot) {
        const float s_value = st[kt][e0 + slot];
        const float p = s_value == -INFINITY ? 0.0F : expf(s_value - new_max);
        partial_sum += p;
        const __bf16 h = static_cast<__bf16>(p);
        ph[slot] = h;
        pl[slot] = static_cast<__bf16>(p - static_cast<float>(h));
      }
      // keys of this k-step for this lane: base + {0..3} and base + 8 + {0..3}
      const int key_base = kt * 32 + (e0 >> 2) * 8 + half * 4;
#pragma unroll
      for (int t = 0; t < kDTiles; ++t) {
        const int d = t * 32 + col;
        const uint16_t *vh_row = &v_s[0][d * kVStride + key_base];
        const uint16_t *vl_row = &v_s[1][d * kVStride + key_base];
        const uint2 h0 = *reinterpret_cast<const uint2 *>(vh_row);
        const uint2 h1 = *reinterpret_cast<const uint2 *>(vh_row + 8);
        const uint2 l0 = *reinterpret_cast<const uint2 *>(vl_row);
        const uint2 l1 = *reinterpret_cast<const uint2 *>(vl_row + 8);
        const uint4 hv = make_uint4(h0.x, h0.y, h1.x, h1.y);
        const uint4 lv = make_uint4(l0.x, l0.y, l1.x, l1.y);
        const bf16x8 vh = __builtin_bit_cast(bf16x8, hv);
        const bf16x8 vl = __builtin_bit_cast(bf16x8, lv);
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
    const uint16_t *__restrict__ v_cache, size_t cache_plane, size_t rows, size_t prefix,
    size_t heads, O out) {
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
      v_s[i] = ok ? get_split(v_cache, v_cache + cache_plane, g) : 0.0F;
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

template <typename O>
Status launch_attention(const uint16_t *q, size_t q_plane, const uint16_t *k_cache,
                        const uint16_t *v_cache, size_t cache_plane, size_t rows,
                        size_t prefix, size_t heads, size_t head_dim, O out,
                        hipStream_t stream) {
  const dim3 mfma_grid(ceil_div(rows, 4 * kQueriesPerWave), static_cast<unsigned>(heads));
  switch (head_dim) {
  case 16:
    hipLaunchKernelGGL((attention_kernel<16, O>), dim3(ceil_div(rows, 64), heads), dim3(256),
                       0, stream, q, q_plane, k_cache, v_cache, cache_plane, rows, prefix,
                       heads, out);
    return launch_status("attention_kernel");
  case 32:
    hipLaunchKernelGGL((flash_attention_kernel<32, O>), mfma_grid, dim3(256), 0, stream, q,
                       q_plane, k_cache, v_cache, cache_plane, rows, prefix, heads, out);
    break;
  case 64:
    hipLaunchKernelGGL((flash_attention_kernel<64, O>), mfma_grid, dim3(256), 0, stream, q,
                       q_plane, k_cache, v_cache, cache_plane, rows, prefix, heads, out);
    break;
  case 128:
    hipLaunchKernelGGL((flash_attention_kernel<128, O>), mfma_grid, dim3(256), 0, stream, q,
                       q_plane, k_cache, v_cache, cache_plane, rows, prefix, heads, out);
    break;
  default:
    return {ErrorCode::kUnsupported,
            "causal_attention: head_dim must be 16, 32, 64 or 128"};
  }
  return launch_status("flash_attention_kernel");
}

}  // namespace

Status qkv_rope(const float *projected, size_t rows, size_t width, size_t heads,
                bool column_split, const float *inv_freq, float rope_scale,
                size_t prefix, uint16_t *q, size_t q_plane, uint16_t *k_cache,
                uint16_t *v_cache, size_t cache_plane, hipStream_t stream) {
  if (projected == nullptr || inv_freq == nullptr || q == nullptr ||
      k_cache == nullptr || v_cache == nullptr || rows == 0 || heads == 0 ||
      width % heads != 0 || (width / heads) % 2 != 0 || !(rope_scale > 0.0F) ||
      q_plane < rows * width || cache_plane < (prefix + rows) * width)
    return {ErrorCode::kInvalidArgument, "qkv_rope: invalid arguments"};
  const size_t n = rows * heads * (width / heads / 2);
  const unsigned grid = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 16384));
  hipLaunchKernelGGL(qkv_rope_kernel, dim3(grid), dim3(256), 0, stream, projected, rows,
                     width, heads, width / heads, column_split ? 1 : 0, inv_freq,
                     rope_scale, prefix, q, q_plane, k_cache, v_cache, cache_plane);
  return launch_status("qkv_rope_kernel");
}

Status causal_attention(const uint16_t *q, size_t q_plane, const uint16_t *k_cache,
                        const uint16_t *v_cache, size_t cache_plane, size_t rows,
                        size_t prefix, size_t heads, size_t head_dim, float *out_f32,
                        uint16_t *out_hi, uint16_t *out_lo, hipStream_t stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      (out_f32 == nullptr && out_hi == nullptr) || rows == 0 || heads == 0 ||
      heads > 65535 || q_plane < rows * heads * head_dim ||
      cache_plane < (prefix + rows) * heads * head_dim)
    return {ErrorCode::kInvalidArgument, "causal_attention: invalid arguments"};
  if (out_f32 != nullptr)
    return launch_attention(q, q_plane, k_cache, v_cache, cache_plane, rows, prefix, heads,
                            head_dim, out_f32, stream);
  return launch_attention(q, q_plane, k_cache, v_cache, cache_plane, rows, prefix, heads,
                          head_dim, SplitOut{out_hi, out_lo}, stream);
}

}  // namespace evo::hip
