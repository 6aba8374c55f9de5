// SPDX-License-Identifier: Apache-2.0
// Attention block of StripedHyena2 on gfx950 (prefill).
//
// qkv_rope: splits the Wqkv projection (head-major `column_split` layout
// [h][q,k,v][d], or component-major [q,k,v][h][d]), applies GPT-NeoX
// half-pair RoPE at position (prefix + row) / rope_scale and appends K/V to
// the resident caches. Reference: evo.cpp `src/cpu/model.cpp:455-509`.
//
// causal_attention: softmax(q.k / sqrt(d)) v over keys [0, position], F32.
// One 256-thread block = 64 queries of one head; four lanes share a query
// (each holds head_dim/4 of q and of the output). K/V tiles of 64 keys are
// staged in LDS; the 64 scores of a tile are kept in registers so the running
// maximum is corrected once per tile (online softmax). Reference semantics:
// `src/cpu/model.cpp:510-544` (full softmax; same value up to F32 rounding).
#include "common.hpp"
#include "ops.hpp"

namespace evo::hip {
namespace {

__global__ void qkv_rope_kernel(const float *__restrict__ projected, size_t rows,
                                size_t width, size_t heads, size_t head_dim,
                                int column_split, const float *__restrict__ inv_freq,
                                float rope_scale, size_t prefix,
                                float *__restrict__ q, float *__restrict__ k_cache,
                                float *__restrict__ v_cache) {
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
    const size_t base_out = head * head_dim;
    {
      const float first = src[source(0, pair)], second = src[source(0, half + pair)];
      q[row * width + base_out + pair] = first * cosine - second * sine;
      q[row * width + base_out + half + pair] = second * cosine + first * sine;
    }
    {
      const float first = src[source(1, pair)], second = src[source(1, half + pair)];
      float *k = k_cache + (prefix + row) * width + base_out;
      k[pair] = first * cosine - second * sine;
      k[half + pair] = second * cosine + first * sine;
    }
    float *v = v_cache + (prefix + row) * width + base_out;
    v[pair] = src[source(2, pair)];
    v[half + pair] = src[source(2, half + pair)];
  }
}

template <int kDim, typename O>  // head_dim, output type
__global__ __launch_bounds__(256) void attention_kernel(
    const float *__restrict__ q, const float *__restrict__ k_cache,
    const float *__restrict__ v_cache, size_t rows, size_t prefix,
    size_t heads, O out) {
  constexpr int kQ = 64, kKeys = 64, kPart = kDim / 4;
  __shared__ float k_s[kKeys * kDim];
  __shared__ float v_s[kKeys * kDim];
  const size_t width = heads * kDim;
  const int tid = threadIdx.x;
  const int qi = tid >> 2, part = tid & 3;
  const size_t head = blockIdx.y;
  const size_t row = blockIdx.x * static_cast<size_t>(kQ) + qi;
  const bool active = row < rows;
  const size_t position = prefix + row;  // last key this query sees
  const float scale = 1.0F / sqrtf(static_cast<float>(kDim));
  float qv[kPart], acc[kPart];
#pragma unroll
  for (int d = 0; d < kPart; ++d) {
    qv[d] = active ? q[row * width + head * kDim + part * kPart + d] : 0.0F;
    acc[d] = 0.0F;
  }
  float running_max = -INFINITY, denominator = 0.0F;
  const size_t last_row = min(rows, blockIdx.x * static_cast<size_t>(kQ) + kQ) - 1;
  const size_t keys_needed = prefix + last_row + 1;
  for (size_t k0 = 0; k0 < keys_needed; k0 += kKeys) {
    __syncthreads();
    for (int i = tid; i < kKeys * kDim / 4; i += 256) {
      const int key = (i * 4) / kDim, d = (i * 4) % kDim;
      float4 kv = make_float4(0, 0, 0, 0), vv = make_float4(0, 0, 0, 0);
      if (k0 + key < keys_needed) {
        kv = *reinterpret_cast<const float4 *>(k_cache + (k0 + key) * width + head * kDim + d);
        vv = *reinterpret_cast<const float4 *>(v_cache + (k0 + key) * width + head * kDim + d);
      }
      *reinterpret_cast<float4 *>(k_s + key * kDim + d) = kv;
      *reinterpret_cast<float4 *>(v_s + key * kDim + d) = vv;
    }
    __syncthreads();
    float scores[kKeys];
    float tile_max = -INFINITY;
#pragma unroll
    for (int j = 0; j < kKeys; ++j) {
      float dot = 0.0F;
#pragma unroll
      for (int d = 0; d < kPart; ++d)
        dot += qv[d] * k_s[j * kDim + part * kPart + d];
      dot += __shfl_xor(dot, 1, 64);
      dot += __shfl_xor(dot, 2, 64);
      const bool visible = k0 + j <= position;
      scores[j] = visible ? dot * scale : -INFINITY;
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
    for (int j = 0; j < kKeys; ++j) {
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

}  // namespace

Status qkv_rope(const float *projected, size_t rows, size_t width, size_t heads,
                bool column_split, const float *inv_freq, float rope_scale,
                size_t prefix, float *q, float *k_cache, float *v_cache,
                hipStream_t stream) {
  if (projected == nullptr || inv_freq == nullptr || q == nullptr ||
      k_cache == nullptr || v_cache == nullptr || rows == 0 || heads == 0 ||
      width % heads != 0 || (width / heads) % 2 != 0 || !(rope_scale > 0.0F))
    return {ErrorCode::kInvalidArgument, "qkv_rope: invalid arguments"};
  const size_t n = rows * heads * (width / heads / 2);
  const unsigned grid = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 16384));
  hipLaunchKernelGGL(qkv_rope_kernel, dim3(grid), dim3(256), 0, stream, projected,
                     rows, width, heads, width / heads, column_split ? 1 : 0,
                     inv_freq, rope_scale, prefix, q, k_cache, v_cache);
  return launch_status("qkv_rope_kernel");
}

template <typename O>
Status launch_attention(const float *q, const float *k_cache, const float *v_cache,
                        size_t rows, size_t prefix, size_t heads, size_t head_dim, O out,
                        hipStream_t stream) {
  const dim3 grid(ceil_div(rows, 64), static_cast<unsigned>(heads));
  switch (head_dim) {
  case 16:
    hipLaunchKernelGGL((attention_kernel<16, O>), grid, dim3(256), 0, stream, q, k_cache,
                       v_cache, rows, prefix, heads, out);
    break;
  case 32:
    hipLaunchKernelGGL((attention_kernel<32, O>), grid, dim3(256), 0, stream, q, k_cache,
                       v_cache, rows, prefix, heads, out);
    break;
  case 64:
    hipLaunchKernelGGL((attention_kernel<64, O>), grid, dim3(256), 0, stream, q, k_cache,
                       v_cache, rows, prefix, heads, out);
    break;
  case 128:
    hipLaunchKernelGGL((attention_kernel<128, O>), grid, dim3(256), 0, stream, q, k_cache,
                       v_cache, rows, prefix, heads, out);
    break;
  default:
    return {ErrorCode::kUnsupported,
            "causal_attention: head_dim must be 16, 32, 64 or 128"};
  }
  return launch_status("attention_kernel");
}

Status causal_attention(const float *q, const float *k_cache,
                        const float *v_cache, size_t rows, size_t prefix,
                        size_t heads, size_t head_dim, float *out_f32,
                        uint16_t *out_hi, uint16_t *out_lo, hipStream_t stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      (out_f32 == nullptr && out_hi == nullptr) || rows == 0 || heads == 0 ||
      heads > 65535)
    return {ErrorCode::kInvalidArgument, "causal_attention: invalid arguments"};
  if (out_f32 != nullptr)
    return launch_attention(q, k_cache, v_cache, rows, prefix, heads, head_dim, out_f32,
                            stream);
  return launch_attention(q, k_cache, v_cache, rows, prefix, heads, head_dim,
                          SplitOut{out_hi, out_lo}, stream);
}

}  // namespace evo::hip
