// SPDX-License-Identifier: Apache-2.0
// Embedding gather, RMSNorm and FIR-history maintenance.
//
// RMSNorm follows evo.cpp `src/cpu_reference.cpp:61-98` /
// `src/cpu/model.cpp:316-334`: y = x / (sqrt(mean(x^2)) + eps) * scale, the
// epsilon added after the square root. One 256-thread block per row; each
// thread reads 16-byte vectors, the sum of squares is reduced with wave
// shuffles and one LDS exchange (F32 throughout).
#include "common.hpp"
#include "row_norm.hpp"
#include "ops.hpp"

namespace evo::hip {
namespace {

// Token ids outside the vocabulary produce zero rows and raise *invalid.
__global__ void embed_kernel(const uint32_t *__restrict__ tokens, size_t rows,
                             const uint16_t *__restrict__ table, size_t vocab,
                             size_t width, float *__restrict__ out,
                             int *__restrict__ invalid) {
  const size_t n = rows * width;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
       i < n; i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t row = i / width, col = i % width;
    const uint32_t token = tokens[row];
    if (token >= vocab) {
      out[i] = 0.0F;
      atomicOr(invalid, 1);
      continue;
    }
    out[i] = bf16_to_f32(table[static_cast<size_t>(token) * width + col]);
  }
}

__global__ __launch_bounds__(256) void rms_norm_kernel(
    const float *__restrict__ x, size_t width, const float *__restrict__ scale,
    float eps, float *__restrict__ out, uint16_t *__restrict__ out_hi,
    uint16_t *__restrict__ out_lo, uint8_t *__restrict__ codes, float code_scale) {
  __shared__ float partial[4];
  const size_t row = blockIdx.x;
  const float *src = x + row * width;
  float sum = 0.0F;
  const bool vec = (width % 4) == 0;
  if (vec) {
    for (size_t c = threadIdx.x * 4; c < width; c += 256 * 4)
      sum = norm_square_sum(*reinterpret_cast<const float4 *>(src + c), sum);
  } else {
    for (size_t c = threadIdx.x; c < width; c += 256)
      sum = fmaf(src[c], src[c], sum);
  }
  const float denominator = norm_denominator(sum, width, eps, partial);
  if (vec) {
    // Four values per thread per pass: 16-byte F32 and 8-byte plane stores,
    // 4-byte code stores.
    for (size_t c = threadIdx.x * 4; c < width; c += 256 * 4) {
      const float4 v = *reinterpret_cast<const float4 *>(src + c);
      const float4 g = *reinterpret_cast<const float4 *>(scale + c);
      const float y[4] = {norm_value(v.x, denominator, g.x), norm_value(v.y, denominator, g.y),
                          norm_value(v.z, denominator, g.z), norm_value(v.w, denominator, g.w)};
      const size_t index = row * width + c;
      if (out != nullptr)
        *reinterpret_cast<float4 *>(out + index) = make_float4(y[0], y[1], y[2], y[3]);
      uint16_t hi[4], lo[4];
      uint8_t code[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = f32_to_bf16(y[e]);
        lo[e] = f32_to_bf16(y[e] - bf16_to_f32(hi[e]));
        code[e] = encode_e4m3(bf16_to_f32(hi[e]) * code_scale);
      }
      if (out_hi != nullptr)
        *reinterpret_cast<uint2 *>(out_hi + index) = __builtin_bit_cast(uint2, hi);
      if (out_lo != nullptr)
        *reinterpret_cast<uint2 *>(out_lo + index) = __builtin_bit_cast(uint2, lo);
      if (codes != nullptr)
        *reinterpret_cast<uint32_t *>(codes + index) = __builtin_bit_cast(uint32_t, code);
    }
    return;
  }
  const SplitOut planes{out_hi, out_lo};
  for (size_t c = threadIdx.x; c < width; c += 256) {
    const float value = norm_value(src[c], denominator, scale[c]);
    const size_t index = row * width + c;
    if (out != nullptr)
      out[index] = value;
    if (out_hi != nullptr)
      put(planes, index, value);
    if (codes != nullptr)
      codes[index] = encode_e4m3(round_bf16(value) * code_scale);
  }
}

// Register-resident variant for width % 4 == 0 and width <= 1024 * kVec: the
// row is read once (kVec 16-byte vectors per thread stay in registers), the
// same per-thread and shuffle reduction order as rms_norm_kernel, and
// non-temporal stores (the outputs feed the next kernel from HBM anyway).
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned u32x2v __attribute__((ext_vector_type(2)));

// Row source of the fused form: x = sum_s part[s] (s in order) (+ bf16
// bias) (+ residual), the split-K reduction's values, also written to
// `sum`; part == nullptr: x is read from memory.
struct NormPartials {
  const float *part;
  int splits;
  size_t plane;
  const uint16_t *bias;
  const float *residual;
  float *sum;
};

template <int kVec, bool kPartials = false>
__global__ __launch_bounds__(256) void rms_norm_reg_kernel(
    const float *__restrict__ x, size_t width, const float *__restrict__ scale,
    float eps, float *__restrict__ out, uint16_t *__restrict__ out_hi,
    uint16_t *__restrict__ out_lo, uint8_t *__restrict__ codes, float code_scale,
    const NormPartials parts) {
  __shared__ float partial[4];
  const size_t row = blockIdx.x;
  const float *src = x + row * width;
  float4 v[kVec];
  float sum = 0.0F;
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const size_t c = threadIdx.x * 4 + j * 1024;
    if constexpr (kPartials) {
      if (c < width) {
        const size_t index = row * width + c;
        float4 acc = *reinterpret_cast<const float4 *>(parts.part + index);
        for (int sp = 1; sp < parts.splits; ++sp) {
          const float4 p = *reinterpret_cast<const float4 *>(parts.part + sp * parts.plane + index);
          acc = make_float4(acc.x + p.x, acc.y + p.y, acc.z + p.z, acc.w + p.w);
        }
        if (parts.bias != nullptr) {
          const uint2 b = *reinterpret_cast<const uint2 *>(parts.bias + c);
          acc = make_float4(acc.x + __builtin_bit_cast(float, b.x << 16),
                            acc.y + __builtin_bit_cast(float, b.x & 0xffff0000U),
                            acc.z + __builtin_bit_cast(float, b.y << 16),
                            acc.w + __builtin_bit_cast(float, b.y & 0xffff0000U));
        }
        if (parts.residual != nullptr) {
          const float4 r = *reinterpret_cast<const float4 *>(parts.residual + index);
          acc = make_float4(acc.x + r.x, acc.y + r.y, acc.z + r.z, acc.w + r.w);
        }
        *reinterpret_cast<float4 *>(parts.sum + index) = acc;
        v[j] = acc;
      } else {
        v[j] = make_float4(0, 0, 0, 0);
      }
    } else {
      v[j] = c < width ? *reinterpret_cast<const float4 *>(src + c) : make_float4(0, 0, 0, 0);
    }
    if (c < width)
      sum = norm_square_sum(v[j], sum);
  }
  const float denominator = norm_denominator(sum, width, eps, partial);
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const size_t c = threadIdx.x * 4 + j * 1024;
    if (c >= width)
      break;
    const float4 g = *reinterpret_cast<const float4 *>(scale + c);
    const float y[4] = {norm_value(v[j].x, denominator, g.x), norm_value(v[j].y, denominator, g.y),
                        norm_value(v[j].z, denominator, g.z), norm_value(v[j].w, denominator, g.w)};
    const size_t index = row * width + c;
    if (out != nullptr) {
      const f32x4v o = {y[0], y[1], y[2], y[3]};
      __builtin_nontemporal_store(o, reinterpret_cast<f32x4v *>(out + index));
    }
    uint16_t hi[4], lo[4];
    uint8_t code[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hi[e] = f32_to_bf16(y[e]);
      lo[e] = f32_to_bf16(y[e] - bf16_to_f32(hi[e]));
      code[e] = encode_e4m3(bf16_to_f32(hi[e]) * code_scale);
    }
    if (out_hi != nullptr)
      __builtin_nontemporal_store(__builtin_bit_cast(u32x2v, hi),
                                  reinterpret_cast<u32x2v *>(out_hi + index));
    if (out_lo != nullptr)
      __builtin_nontemporal_store(__builtin_bit_cast(u32x2v, lo),
                                  reinterpret_cast<u32x2v *>(out_lo + index));
    if (codes != nullptr)
      __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, code),
                                  reinterpret_cast<uint32_t *>(codes + index));
  }
}

// history[h, c] <- row h of the last H rows of [history ; x]. Each thread owns
// one channel and walks h upwards, so an old row is read before it is
// overwritten (it only moves to a lower index).
__global__ void update_history_kernel(const float *__restrict__ x, size_t rows,
                                      size_t channels, float *history,
                                      size_t history_rows) {
  const size_t c = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (c >= channels)
    return;
  for (size_t h = 0; h < history_rows; ++h) {
    const size_t source = h + rows;  // index into [history ; x]
    history[h * channels + c] = source < history_rows
                                    ? history[source * channels + c]
                                    : x[(source - history_rows) * channels + c];
  }
}

}  // namespace

Status embed_tokens(const uint32_t *tokens, size_t rows, const uint16_t *table,
                    size_t vocab, size_t width, float *out, int *invalid,
                    hipStream_t stream) {
  if (tokens == nullptr || table == nullptr || out == nullptr || invalid == nullptr ||
      rows == 0 || width == 0)
    return {ErrorCode::kInvalidArgument, "embed_tokens: invalid arguments"};
  const size_t n = rows * width;
  const unsigned grid = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 16384));
  hipLaunchKernelGGL(embed_kernel, dim3(grid), dim3(256), 0, stream, tokens, rows,
                     table, vocab, width, out, invalid);
  return launch_status("embed_kernel");
}

Status rms_norm(const float *x, size_t rows, size_t width, const float *scale,
                float eps, float *out, uint16_t *out_hi, uint16_t *out_lo,
                hipStream_t stream, uint8_t *codes, float code_scale) {
  if (x == nullptr || scale == nullptr ||
      (out == nullptr && out_hi == nullptr && codes == nullptr) || rows == 0 ||
      width == 0 || rows > (1U << 31) ||
      (codes != nullptr && !(code_scale > 0.0F && __builtin_isfinite(code_scale))))
    return {ErrorCode::kInvalidArgument, "rms_norm: invalid arguments"};
  const dim3 grid(static_cast<unsigned>(rows)), block(256);
  const NormPartials none{nullptr, 0, 0, nullptr, nullptr, nullptr};
  if (width % 4 == 0 && width <= 2048)
    hipLaunchKernelGGL(rms_norm_reg_kernel<2>, grid, block, 0, stream, x, width, scale, eps,
                       out, out_hi, out_lo, codes, code_scale, none);
  else if (width % 4 == 0 && width <= 4096)
    hipLaunchKernelGGL(rms_norm_reg_kernel<4>, grid, block, 0, stream, x, width, scale, eps,
                       out, out_hi, out_lo, codes, code_scale, none);
  else if (width % 4 == 0 && width <= 8192)
    hipLaunchKernelGGL(rms_norm_reg_kernel<8>, grid, block, 0, stream, x, width, scale, eps,
                       out, out_hi, out_lo, codes, code_scale, none);
  else
    hipLaunchKernelGGL(rms_norm_kernel, grid, block, 0, stream, x, width, scale, eps, out,
                       out_hi, out_lo, codes, code_scale);
  return launch_status("rms_norm_kernel");
}

Status rms_norm_partials(const SplitPartials &src, float *sum, size_t rows, size_t width,
                         const float *scale, float eps, uint16_t *out_hi, uint16_t *out_lo,
                         hipStream_t stream, uint8_t *codes, float code_scale) {
  if (src.splits == 0)
    return rms_norm(sum, rows, width, scale, eps, nullptr, out_hi, out_lo, stream, codes,
                    code_scale);
  const bool aligned = width % 4 == 0 && reinterpret_cast<uintptr_t>(src.part) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(sum) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(src.residual) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(src.bias) % 8 == 0;
  if (!aligned || width > 8192 || src.plane != rows * width) {
    // Unfused: the reduction, then the norm of what it wrote.
    EVO_TRY(split_k_finish(src, sum, rows, width, stream));
    return rms_norm(sum, rows, width, scale, eps, nullptr, out_hi, out_lo, stream, codes,
                    code_scale);
  }
  if (scale == nullptr || sum == nullptr || (out_hi == nullptr && codes == nullptr) ||
      rows == 0 || rows > (1U << 31) ||
      (codes != nullptr && !(code_scale > 0.0F && __builtin_isfinite(code_scale))))
    return {ErrorCode::kInvalidArgument, "rms_norm_partials: invalid arguments"};
  const dim3 grid(static_cast<unsigned>(rows)), block(256);
  const NormPartials parts{src.part, src.splits, src.plane, src.bias, src.residual, sum};
  if (width <= 2048)
    hipLaunchKernelGGL((rms_norm_reg_kernel<2, true>), grid, block, 0, stream, nullptr, width,
                       scale, eps, nullptr, out_hi, out_lo, codes, code_scale, parts);
  else if (width <= 4096)
    hipLaunchKernelGGL((rms_norm_reg_kernel<4, true>), grid, block, 0, stream, nullptr, width,
                       scale, eps, nullptr, out_hi, out_lo, codes, code_scale, parts);
  else
    hipLaunchKernelGGL((rms_norm_reg_kernel<8, true>), grid, block, 0, stream, nullptr, width,
                       scale, eps, nullptr, out_hi, out_lo, codes, code_scale, parts);
  return launch_status("rms_norm_reg_kernel (split-K partials)");
}

namespace {
__global__ __launch_bounds__(256) void zero_regions_kernel(const ZeroRegion *__restrict__ regions) {
  const ZeroRegion r = regions[blockIdx.y];
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < r.words;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    r.ptr[i] = 0U;
}
}  // namespace

Status zero_regions(const ZeroRegion *regions, size_t count, size_t max_words,
                    hipStream_t stream) {
  if (count == 0 || max_words == 0)
    return Status::Ok();
  if (regions == nullptr || count > 65535)
    return {ErrorCode::kInvalidArgument, "zero_regions: invalid arguments"};
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>(ceil_div(max_words, 256), 64));
  hipLaunchKernelGGL(zero_regions_kernel, dim3(blocks, static_cast<unsigned>(count)), dim3(256),
                     0, stream, regions);
  return launch_status("zero_regions_kernel");
}

Status update_history(const float *x, size_t rows, size_t channels,
                      float *history, size_t history_rows, float *scratch,
                      hipStream_t stream) {
  (void)scratch;
  if (history_rows == 0)
    return Status::Ok();
  if (x == nullptr || history == nullptr || rows == 0 || channels == 0)
    return {ErrorCode::kInvalidArgument, "update_history: invalid arguments"};
  hipLaunchKernelGGL(update_history_kernel, dim3(ceil_div(channels, 256)), dim3(256),
                     0, stream, x, rows, channels, history, history_rows);
  return launch_status("update_history_kernel");
}

}  // namespace evo::hip
