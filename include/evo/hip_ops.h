/* SPDX-License-Identifier: Apache-2.0
 *
 * Operator-level C ABI of libevo_hip.so: the gfx950 kernels of the
 * StripedHyena2 prefill path on caller-owned device memory.
 *
 * All pointers are device pointers (hipMalloc'd or a torch tensor's
 * data_ptr()); `stream` is a hipStream_t (NULL = the default stream). Calls
 * are asynchronous on that stream and never allocate device memory: every
 * temporary lives in a caller-provided workspace whose size the matching
 * *_workspace_bytes query returns. Shapes are validated on the host before
 * any launch; invalid arguments return EVO_STATUS_INVALID_ARGUMENT with the
 * message in evo_last_error(). BF16 tensors are raw uint16 bit patterns.
 *
 * Each entry point names the reference interface it replaces.
 */
#ifndef EVO_HIP_OPS_H
#define EVO_HIP_OPS_H

#include <stddef.h>
#include <stdint.h>

#include "evo/evo.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Whole-sequence prefill with tokens (uint32 [count]) and logits (F32
 * [count, vocab]) in device memory, for callers that keep the stream on the
 * GPU (serving loops, benchmarks): same chunk loop, caches and numerics as
 * evo_context_prefill, but no host copies; synchronises the context stream
 * once at the end. The context is reset first (position 0), so one context can
 * serve successive sequences. Token ids >= vocab fail the call.
 * Replaces the CUDA `PipelineModel::prefill` loop driven from
 * `src/c_api.cpp:962-989`, minus the host logits. */
EVO_API evo_status evo_hip_context_prefill_resident(evo_context *context,
                                                    const uint32_t *tokens,
                                                    size_t count, float *logits);
/* The context's HIP stream (hipStream_t), for ordering caller work. */
EVO_API void *evo_hip_context_stream(const evo_context *context);

/* Measurement hooks (no counterpart in the reference): with timing on, each
 * prefill records HIP events on the context stream around every layer's MLP
 * l1/l2 product (the dominant kernel); evo_hip_context_product_time returns
 * the summed duration (ms) and the number of launches of the last chunk
 * prefilled, once the caller has seen that prefill complete. Off by default. */
EVO_API evo_status evo_hip_context_set_product_timing(evo_context *context, int enable);
EVO_API evo_status evo_hip_context_product_time(const evo_context *context, float *ms,
                                                size_t *launches);

/* Storage type of activation tensors passed to the Hyena operator. */
/* EVO_HIP_SPLIT: F32 input, output as split BF16 planes [2][rows][cols]
 * (hi = bf16(y), lo = bf16(y - hi)), the GEMM activation layout.
 * EVO_HIP_BF16_SPLIT: BF16 input (the FP8 projection's output), split
 * output; Hyena operator only.
 * EVO_HIP_F16 / EVO_HIP_BF16_F16: F32 / BF16 input, output one FP16 plane
 * [rows][cols], fp16(y) rounded to nearest even and saturated to +-65504
 * (the activation of the one-pass FP16 out-projection); Hyena operator
 * only. */
typedef enum evo_hip_dtype {
  EVO_HIP_F32 = 0,
  EVO_HIP_BF16 = 1,
  EVO_HIP_SPLIT = 2,
  EVO_HIP_BF16_SPLIT = 3,
  EVO_HIP_F16 = 4,
  EVO_HIP_BF16_F16 = 5,
  /* OR-ed into the Hyena operator's dtype: the projection holds stream s
   * (x2, x1, v) of channel c at column s*W + c instead of the reference's
   * 3c + s (the library permutes its projection weights this way). */
  EVO_HIP_PLANAR = 0x100,
  /* OR-ed into the Hyena operator's dtype: every inner_filter tap is a BF16
   * value (evo2 artifacts store `filter.h` as BF16), which lets the HCM
   * operator form its Toeplitz product in two MFMA passes instead of three
   * (same result). */
  EVO_HIP_BF16_TAPS = 0x200
} evo_hip_dtype;
typedef enum evo_hip_hyena_kind {
  EVO_HIP_HYENA_HCS = 0,
  EVO_HIP_HYENA_HCM = 1,
  EVO_HIP_HYENA_HCL = 2
} evo_hip_hyena_kind;

/* Fused Hyena mixer of one block: short FIR (short_len taps, per column of
 * the [L, 3W] projection with interleaved (x2, x1, v) triples), u = x1*v, the
 * long filter (HCS grouped FIR / HCM grouped causal conv + D*u / HCL modal
 * recurrence + D*u), times x2; output [L, W] in `dtype`.
 * Replaces evo.cpp `bf16_fir_prefill_direct` + `bf16_hcs_prefill` /
 * `bf16_hcm_prefill` / `bf16_hcl_prefill`
 * (`include/evo/cuda/hyena.hpp:154-252`) and the CPU mixer
 * (`src/cpu/model.cpp:546-605`).
 *   short_filter  BF16 [3W, short_len]
 *   inner_filter  F32 [groups, inner_len]          (HCS/HCM; else NULL)
 *   direct        F32 [W]                          (HCM/HCL; else NULL)
 *   poles         F32 [W, state] = exp(log_poles)  (HCL; else NULL)
 *   residues      F32 [W, state]                   (HCL; else NULL)
 *   short_history F32 [short_len-1, 3W], inner_history F32 [inner_len-1, W],
 *   modal_state   F32 [W, state]: optional continuation caches (NULL = zero
 *                 initial state, nothing kept); read as the state before row
 *                 0 and overwritten with the state after row L-1. */
EVO_API size_t evo_hip_hyena_workspace_bytes(evo_hip_hyena_kind kind,
                                             size_t length, size_t width,
                                             size_t state_size);
EVO_API evo_status evo_hip_hyena_forward(
    evo_hip_hyena_kind kind, evo_hip_dtype dtype, const void *projection,
    size_t length, size_t width, const uint16_t *short_filter,
    size_t short_len, const float *inner_filter, size_t groups,
    size_t inner_len, const float *direct, const float *poles,
    const float *residues, size_t state_size, float *short_history,
    float *inner_history, float *modal_state, void *workspace,
    size_t workspace_bytes, void *output, void *stream);

/* Allocation-free variant of evo_hip_hyena_forward: same arguments minus
 * the workspace, same kernels and results. The workspace comes from a fixed
 * device array of evo_hip_hyena_static_scratch_bytes() (32 MiB) in the
 * library, one per device, held until the process ends; the call fails with
 * EVO_STATUS_INVALID_ARGUMENT, before any launch, when the path the shape
 * takes keeps more than that in its workspace. Only two paths use one: the
 * three-pass HCL fallback (planar projections, short filters other than 3
 * taps, W % 16 != 0; chunk states of evo_hip_hyena_workspace_bytes()) and
 * the F32-tap HCS/HCM MFMA FIR (its Toeplitz table, 2.6 MB at W = 4096).
 * The model's shapes (one-pass HCL, streaming HCS/HCM) need none and are
 * accepted at any length.
 * The call makes no device allocation (no hipMalloc/hipFree), so callers that
 * cannot allocate (code under HIP graph capture, tight serving loops) can
 * use it. Every call on a device shares that device's array: calls that
 * overlap on one device (different streams, threads) race; serialise them.
 * No counterpart in the reference: evo.cpp's operators always receive their
 * scratch from the caller or allocate it. */
EVO_API size_t evo_hip_hyena_static_scratch_bytes(void);
EVO_API evo_status evo_hip_hyena_forward_static(
    evo_hip_hyena_kind kind, evo_hip_dtype dtype, const void *projection,
    size_t length, size_t width, const uint16_t *short_filter,
    size_t short_len, const float *inner_filter, size_t groups,
    size_t inner_len, const float *direct, const float *poles,
    const float *residues, size_t state_size, float *short_history,
    float *inner_history, float *modal_state, void *output, void *stream);

/* codes[i] = E4M3FN(float(bf16(x[i])) * scale), RNE, satfinite.
 * Replaces `software_e4m3_quantize_bf16_codes` (`include/evo/cuda/ops.hpp:92-96`). */
EVO_API evo_status evo_hip_e4m3_quantize(evo_hip_dtype dtype, const void *x,
                                         size_t count, float scale,
                                         uint8_t *codes, void *stream);

/* Software-FP8 projection out[M,N] = bf16(QGMMA(in_codes[M,K], w_codes[N,K])
 * * output_scale), stored as F32. mode 0 = E4M3 MFMA with promotion every 32
 * K, 1 = every 128 K, 2 = bit-exact integer QGMMA emulation.
 * Replaces `software_e4m3_h100_linear` (`include/evo/cuda/ops.hpp:104-114`). */
EVO_API evo_status evo_hip_fp8_linear(const uint8_t *in_codes,
                                      const uint8_t *w_codes, float *out,
                                      size_t m, size_t n, size_t k,
                                      float output_scale, int mode,
                                      void *stream);

/* The same product stored as BF16 [M,N] (the projection's own output type:
 * each value already is bf16(acc * output_scale)). */
EVO_API evo_status evo_hip_fp8_linear_bf16(const uint8_t *in_codes,
                                           const uint8_t *w_codes, uint16_t *out,
                                           size_t m, size_t n, size_t k,
                                           float output_scale, int mode, void *stream);

/* GEMM activation layout: hi[i] = bf16(x[i]), lo[i] = bf16(x[i] - hi[i])
 * (lo may be NULL for BF16-only activations). */
EVO_API evo_status evo_hip_split_f32(const float *x, size_t count, uint16_t *hi,
                                     uint16_t *lo, void *stream);

/* out[M,N] = x[M,K] . w[N,K]^T (+ bf16 bias[N]) (+ residual[M,N]); x as
 * split BF16 planes (x_lo NULL: one BF16 MFMA pass), w BF16, out F32.
 * Replaces `bf16_linear` (`include/evo/cuda/ops.hpp:61-70`) and the CPU
 * `linear` (`src/cpu/model.cpp:284-314`). */
EVO_API evo_status evo_hip_linear(const uint16_t *x_hi, const uint16_t *x_lo,
                                  const uint16_t *w, const uint16_t *bias,
                                  const float *residual, size_t m, size_t n,
                                  size_t k, float *out, void *stream);

/* evo_hip_linear with an F32 device workspace (16-byte aligned; otherwise
 * it is not used): launches with few output tiles split K across blocks
 * (partials in the workspace, summed in split order before the epilogue),
 * the path the model takes for short prompts. The same reference interface
 * as evo_hip_linear. */
EVO_API evo_status evo_hip_linear_split(const uint16_t *x_hi, const uint16_t *x_lo,
                                        const uint16_t *w, const uint16_t *bias,
                                        const float *residual, size_t m, size_t n,
                                        size_t k, float *out, float *workspace,
                                        size_t workspace_bytes, void *stream);

/* Gated MLP out[M,W] = l3(act(l1 x) * l2 x) (+ residual) with act = erf-GELU
 * when gelu != 0. w12 is the interleaved [2*Fp, W] l1/l2 weight (32-row
 * blocks, Fp = F rounded up to 32) built by evo_hip_pack_mlp;
 * inner_workspace holds the gated [M, F] activation as split planes
 * (2*M*F uint16, or M*F when x_lo is NULL).
 * Replaces `bf16_mlp` (`include/evo/cuda/ops.hpp:133-138`). */
EVO_API evo_status evo_hip_pack_mlp(const uint16_t *l1, const uint16_t *l2,
                                    size_t inner, size_t width, uint16_t *w12,
                                    void *stream);
EVO_API evo_status evo_hip_gated_mlp(const uint16_t *x_hi, const uint16_t *x_lo,
                                     const uint16_t *w12, const uint16_t *l3,
                                     size_t m, size_t width, size_t inner,
                                     int gelu, uint16_t *inner_workspace,
                                     const float *residual, float *out,
                                     void *stream);

/* RMSNorm y = x / (sqrt(mean(x^2)) + eps) * scale over rows of width,
 * written as F32 (out) and/or split BF16 planes (out_hi, out_lo).
 * Replaces `bf16_rms_norm` (`include/evo/cuda/ops.hpp:117-120`). */
EVO_API evo_status evo_hip_rms_norm(const float *x, size_t rows, size_t width,
                                    const float *scale, float eps, float *out,
                                    uint16_t *out_hi, uint16_t *out_lo,
                                    void *stream);

/* RMSNorm fused with the FP8 projection's input quantisation: codes =
 * E4M3FN(bf16(y) * code_scale) of the normed rows, without writing y
 * (the sequence `bf16_rms_norm` + `quantize_bf16_e4m3` of the reference's
 * FP8 projection path, `src/cuda/ops.cu:72-113, 250-262`). */
EVO_API evo_status evo_hip_rms_norm_e4m3(const float *x, size_t rows, size_t width,
                                         const float *scale, float eps, float code_scale,
                                         uint8_t *codes, void *stream);

/* Few-row products (m <= 4, the decode step) of RMSNorm'd rows without the
 * norm's own launch: each block normalises x [m, k] (F32, 16-byte aligned,
 * scale [k]) itself in the order evo_hip_rms_norm uses, so the results equal
 * evo_hip_rms_norm (split planes when split != 0, else hi only) followed by
 * evo_hip_linear, and evo_hip_rms_norm_e4m3 followed by
 * evo_hip_fp8_linear_bf16 (modes 0 and 1), bit for bit. They fuse the
 * reference's `bf16_rms_norm` with `bf16_linear` / the FP8 projection
 * (`include/evo/cuda/ops.hpp:61-70, 104-120`) for the decode path. */
EVO_API evo_status evo_hip_linear_normed(const float *x, size_t m, size_t k,
                                         const float *scale, float eps, int split,
                                         const uint16_t *w, size_t n, float *out,
                                         void *stream);
EVO_API evo_status evo_hip_fp8_linear_normed(const float *x, size_t m, size_t k,
                                             const float *scale, float eps,
                                             float input_scale, const uint8_t *w_codes,
                                             size_t n, float output_scale, int mode,
                                             uint16_t *out, void *stream);

/* Attention block body: split the Wqkv output [rows, 3W], apply RoPE at
 * positions prefix.., append K/V at `prefix` of the caches, causal softmax
 * attention into out [rows, W] F32. query is workspace of 2*rows*W uint16;
 * key_cache holds split BF16 planes [2][capacity][W] uint16 and value_cache
 * the transposed planes [2][W][capacity], each 16-position block stored in
 * the order 0-3, 8-11, 4-7, 12-15. capacity must be a multiple of 64, and
 * cache entries never written must hold finite values (zero the caches once).
 * Replaces `bf16_split_qkv` + `bf16_apply_rope` + `bf16_kv_append` +
 * `bf16_online_causal_attention` (`include/evo/cuda/attention.hpp:100-133`). */
EVO_API evo_status evo_hip_attention(const float *projected, size_t rows,
                                     size_t width, size_t heads,
                                     int column_split, const float *inv_freq,
                                     float rope_scale, size_t prefix,
                                     uint16_t *query, uint16_t *key_cache,
                                     uint16_t *value_cache, size_t capacity,
                                     float *out, void *stream);

/* evo_hip_attention with an F32 device workspace: a single query (rows == 1,
 * head_dim 32/64/128) is then split over its keys in chunks of 256 (per
 * chunk and head: max, sum and head_dim partial outputs in the workspace),
 * the decode step's path. The same reference interface. */
EVO_API evo_status evo_hip_attention_ws(const float *projected, size_t rows,
                                        size_t width, size_t heads,
                                        int column_split, const float *inv_freq,
                                        float rope_scale, size_t prefix,
                                        uint16_t *query, uint16_t *key_cache,
                                        uint16_t *value_cache, size_t capacity,
                                        float *out, float *workspace,
                                        size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif
