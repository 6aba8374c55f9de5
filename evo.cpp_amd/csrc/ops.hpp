// SPDX-License-Identifier: Apache-2.0
// Host launchers of the gfx950 kernels (device pointers, one HIP stream).
// Each launcher validates shapes on the host before it launches, so no kernel
// runs with a grid its indexing does not cover.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "status.hpp"

namespace evo::hip {

enum GemmEpilogue : int {
  kGemmStore = 0,
  kGemmBias = 1,
  kGemmResidual = 2,
  kGemmBiasResidual = 3,
  kGemmGated = 4,
};

// Output of a producer kernel feeding a GEMM: split BF16 planes
// hi = bf16(v), lo = bf16(v - hi) (lo null: BF16 activations only).
struct SplitOut {
  uint16_t *hi;
  uint16_t *lo;
};

// Output of a producer kernel as one FP16 plane, fp16(v) rounded to nearest
// even and saturated to +-65504, for the one-pass FP16 products. A value
// outside the FP16 range (or NaN) sets bit 1 of *saturated when it is given.
struct F16Out {
  uint16_t *out;
  int *saturated = nullptr;
};
// Bit of the context's device flag that an out-of-range FP16 store raises
// (bit 0: a token outside the vocabulary).
constexpr int kFlagF16Range = 2;

// A GEMM activation as split BF16 planes: hi = bf16(a), lo = bf16(a - hi)
// (lo null: BF16 activations), row stride ld elements.
struct Activation {
  const uint16_t *hi;
  const uint16_t *lo;
  size_t ld;
  bool f16 = false;  // hi holds FP16 bits (lo null) and W is FP16
};
// GEMM output: F32 (store/bias/residual modes) or split planes (gated mode,
// lo may be null), row stride ld elements.
struct GemmOutput {
  float *f32;
  uint16_t *hi;
  uint16_t *lo;
  size_t ld;
};
// RMSNorm of F32 rows x [M][ld] (scale [K], eps after the square root)
// folded into a few-row product (M <= 4) as its input: the product's blocks
// each normalise the rows in the order rms_norm uses, so the result equals
// rms_norm followed by the unfused product, bit for bit, without the norm's
// launch and round trip (decode).
struct RowNorm {
  const float *x;
  const float *scale;
  float eps;
  size_t ld;
};
// Split-K partial products left for their consumer: C[m, n] =
// sum_s part[s][m, n] (s in order) (+ bf16 bias[n]) (+ residual[m, n]),
// C row stride N. splits == 0: nothing is pending.
struct SplitPartials {
  const float *part = nullptr;
  int splits = 0;
  size_t plane = 0;  // floats per partial (M * N)
  const uint16_t *bias = nullptr;
  const float *residual = nullptr;
};
// C = A . W^T with W BF16 [N,K]; see gemm.hip.
// With a split workspace (F32), launches with few output tiles (non-gated
// modes) split K across blocks and sum the partials in split order. With
// `deferred` (and C rows of stride N), such a launch stores only the
// partials and describes them there, for a consumer that sums them itself
// (rms_norm_partials, or split_k_finish); otherwise deferred->splits = 0.
Status gemm_bf16w(const Activation &a, const uint16_t *W, const GemmOutput &out,
                  size_t M, size_t N, size_t K, GemmEpilogue mode,
                  const uint16_t *bias, const float *residual, bool gelu,
                  size_t gated_width, hipStream_t stream, float *split_workspace = nullptr,
                  size_t split_workspace_bytes = 0, SplitPartials *deferred = nullptr);
// Forms C [rows, width] from pending partials (what the GEMM's own
// reduction would have written).
Status split_k_finish(const SplitPartials &src, float *C, size_t rows, size_t width,
                      hipStream_t stream);
// The same product of norm(x) (M <= 4; `split`: the activation as hi + lo
// planes, as the hip-f32 profile's rms_norm writes it, else hi only).
Status gemm_bf16w_normed(const RowNorm &norm, bool split, const uint16_t *W,
                         const GemmOutput &out, size_t M, size_t N, size_t K,
                         GemmEpilogue mode, const uint16_t *bias, const float *residual,
                         bool gelu, size_t gated_width, hipStream_t stream);
// hi[i] = bf16(x[i]), lo[i] = bf16(x[i] - hi[i]) (lo may be null).
// hi + lo (split BF16 planes) -> FP16 bits (RNE, saturating at 65504).
Status planes_to_f16(const uint16_t *hi, const uint16_t *lo, size_t n, uint16_t *out,
                     hipStream_t stream, int *saturated = nullptr);
// BF16 -> FP16 bits (RNE, saturating), e.g. a weight for FP16 products.
Status bf16_to_f16(const uint16_t *x, size_t n, uint16_t *out, hipStream_t stream);
Status split_planes(const float *x, size_t n, uint16_t *hi, uint16_t *lo,
                    hipStream_t stream);

// ---- Software FP8 (fp8.hip).
// codes[i] = E4M3FN_RNE_satfinite(float(bf16(x[i])) * scale).
Status e4m3_quantize_f32(const float *x, size_t n, float scale, uint8_t *codes,
                         hipStream_t stream);
Status e4m3_quantize_bf16(const uint16_t *x, size_t n, float scale,
                          uint8_t *codes, hipStream_t stream);
enum Fp8Mode : int {
  kFp8MfmaK32 = 0,   // E4M3 MFMA, promotion to the E8M13 accumulator every 32 K
  kFp8MfmaK128 = 1,  // E4M3 MFMA, promotion every 128 K
  kFp8Exact = 2,     // integer QGMMA emulation, bit-exact to the reference
};
// out[M,N] (F32 holding BF16 values) = bf16(QGMMA(in_codes, w_codes) * output_scale)
// (+ optional F32 residual added after the BF16 rounding).
Status fp8_linear(const uint8_t *in_codes, const uint8_t *w_codes, float *out,
                  size_t M, size_t N, size_t K, float output_scale,
                  Fp8Mode mode, hipStream_t stream);
// Same product with the BF16 result stored as BF16 (exact: the value already
// is a BF16 number).
Status fp8_linear(const uint8_t *in_codes, const uint8_t *w_codes, uint16_t *out,
                  size_t M, size_t N, size_t K, float output_scale,
                  Fp8Mode mode, hipStream_t stream);
// The MFMA-mode product (M <= 4) of the codes e4m3(bf16(norm(x)) *
// input_scale), which the blocks form themselves (the codes rms_norm writes).
Status fp8_linear_normed(const RowNorm &norm, float input_scale, const uint8_t *w_codes,
                         uint16_t *out, size_t M, size_t N, size_t K, float output_scale,
                         Fp8Mode mode, hipStream_t stream);

// ---- Elementwise / normalisation (elementwise.hip).
Status embed_tokens(const uint32_t *tokens, size_t rows, const uint16_t *table,
                    size_t vocab, size_t width, float *out, int *invalid,
                    hipStream_t stream);
// Writes the F32 result to out_f32 and/or split planes (out_hi, out_lo).
// With codes, also E4M3 codes of bf16(y) * code_scale (the FP8 projection's
// input quantisation fused into the norm).
Status rms_norm(const float *x, size_t rows, size_t width, const float *scale,
                float eps, float *out_f32, uint16_t *out_hi, uint16_t *out_lo,
                hipStream_t stream, uint8_t *codes = nullptr, float code_scale = 1.0F);
// rms_norm of x = the sum of pending split-K partials, which it also
// writes to `sum` (F32 [rows, width]): split_k_finish followed by rms_norm
// of its output, in one pass, with the same values.
Status rms_norm_partials(const SplitPartials &src, float *sum, size_t rows, size_t width,
                         const float *scale, float eps, uint16_t *out_hi, uint16_t *out_lo,
                         hipStream_t stream, uint8_t *codes = nullptr,
                         float code_scale = 1.0F);
// Copies the last `history` rows of the sequence [old_history ; x] into
// history (F32 [history, channels]), keeping continuation caches.
Status update_history(const float *x, size_t rows, size_t channels,
                      float *history, size_t history_rows, float *scratch,
                      hipStream_t stream);
// A device region of `words` 32-bit words for zero_regions.
struct ZeroRegion {
  uint32_t *ptr;
  size_t words;
};
// Clears the `count` regions listed in the device table `regions` (the
// largest `max_words` words long) in one launch.
Status zero_regions(const ZeroRegion *regions, size_t count, size_t max_words,
                    hipStream_t stream);

// ---- Hyena operator (hyena.hip). Projection P [L, 3W] interleaved triples
// (x2, x1, v) per channel. Caches (may be null for a fresh sequence):
// short_history F32 [short_len-1, 3W], inner_history F32 [inner_len-1, W],
// modal_state F32 [W, S]. They are read as the state before row 0 and
// rewritten to the state after row L-1.
enum HyenaKind : int { kHyenaHcs = 0, kHyenaHcm = 1, kHyenaHcl = 2 };
struct HyenaWeights {
  const uint16_t *short_filter;  // BF16 [3W, short_len]
  size_t short_len;
  const float *inner_filter;     // F32 [groups, inner_len] (HCS/HCM)
  size_t groups, inner_len;
  const float *direct;           // F32 [W] (HCM/HCL)
  const float *poles;            // F32 [W, S] = exp(log_poles) (HCL)
  const float *residues;         // F32 [W, S] (HCL)
  size_t state;
  bool taps_bf16;                // every inner tap is a BF16 value (artifact filters)
};
// Size of the fixed device scratch behind the allocation-free Hyena entry
// point, and its address on the current device (resolved once per device).
constexpr size_t kHyenaStaticScratchBytes = size_t{32} << 20;
Status hyena_static_scratch(void **address);
size_t hyena_workspace_bytes(int kind, size_t length, size_t width,
                             size_t state);
// O: float* (F32 out), uint16_t* (BF16 out) or SplitOut (GEMM planes).
// The projection [L, 3W] holds stream s (x2, x1, v) of channel c at column
// 3c + s (the reference layout) or, when planar_projection, at s * W + c.
template <typename T, typename O>
Status hyena_forward(int kind, const T *projection, size_t length,
                     size_t width, bool planar_projection, const HyenaWeights &weights,
                     float *short_history, float *inner_history,
                     float *modal_state, void *workspace,
                     size_t workspace_bytes, O out, hipStream_t stream);

// ---- Attention (attention.hip). Q and the K/V caches are split BF16 planes:
// plane 0 (hi) at the pointer, plane 1 (lo) `*_plane` elements further.
// The key cache is [capacity][W]; the value cache is transposed, V^T
// [W][capacity], each 16-position block stored in the order 0-3, 8-11, 4-7,
// 12-15 (bits 2 and 3 of the position swapped). capacity is a multiple of
// 64 and cache rows never written must hold finite values (zero them once).
// qkv_rope splits the QKV projection [rows, 3W] into rotated Q, rotated K and
// V, appending K/V at position `prefix` of the caches. With v_range_flag, a V
// value outside the FP16 range (or NaN) raises kFlagF16Range there: the
// attention outputs, convex combinations of V, then stay inside it.
Status qkv_rope(const float *projected, size_t rows, size_t width, size_t heads,
                bool column_split, const float *inv_freq, float rope_scale,
                size_t prefix, uint16_t *q, size_t q_plane, uint16_t *k_cache,
                uint16_t *v_cache, size_t cache_plane, size_t capacity, hipStream_t stream,
                int *v_range_flag = nullptr);
// Causal attention of `rows` queries at positions prefix.. against keys
// [0, prefix + rows). Layout [time, heads, head_dim] = [time, W]. Output F32
// (out_f32), split planes (out_hi, out_lo), or with out_f16 one saturated
// FP16 plane in out_hi (its range follows from V's: see qkv_rope).
Status causal_attention(const uint16_t *q, size_t q_plane, const uint16_t *k_cache,
                        const uint16_t *v_cache, size_t cache_plane, size_t capacity,
                        size_t rows, size_t prefix, size_t heads, size_t head_dim,
                        float *out_f32, uint16_t *out_hi, uint16_t *out_lo,
                        hipStream_t stream, float *workspace = nullptr,
                        size_t workspace_bytes = 0, bool out_f16 = false);

}  // namespace evo::hip
