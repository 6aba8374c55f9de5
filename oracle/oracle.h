/* SPDX-License-Identifier: Apache-2.0
 *
 * CPU oracle for the StripedHyena2 prefill path: TEST INFRASTRUCTURE ONLY.
 *
 * This library restates the reference's single-threaded F32 CPU algorithm
 * (evo.cpp `src/cpu/model.cpp:205-714`, `src/cpu_reference.cpp`,
 * `src/fp8.cpp`) and the host QGMMA oracle (`tests/test_cuda_ops.cu:119-187`).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker. The product (libevo_hip.so) never links
 * or calls it.
 *
 * Parity pinning of each function (what fixes its results independently of
 * this restatement) is listed next to its declaration.
 */
#ifndef EVO_ORACLE_H
#define EVO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- E4M3FN codec: src/fp8.cpp:26-68.
 * Pinned by: the 29 PyTorch code vectors of tests/test_fp8.cpp:22-33 and
 * an exhaustive decode->encode round trip over all 254 finite codes. */
uint8_t oracle_e4m3_encode(float value);
float oracle_e4m3_decode(uint8_t code);
/* codes[i] = encode(float(bf16_rne(x[i])) * scale) (src/cuda/ops.cu:250-262
 * applied to an F32 activation first rounded to BF16). */
void oracle_e4m3_quantize_f32(const float *x, size_t n, float scale,
                              uint8_t *codes);
/* codes[i] = encode(float(bf16 bits[i]) * scale). */
void oracle_e4m3_quantize_bf16(const uint16_t *x, size_t n, float scale,
                               uint8_t *codes);

/* ---- H100 QGMMA emulation: tests/test_cuda_ops.cu:119-187 (global
 * alignment per K group incl. accumulator, 13 fractional bits, E8M13
 * truncation), output bf16_rne(acc * output_scale) (src/cuda/ops.cu:436-440).
 * group_k is 32 in the reference; other multiples of 32 are allowed for the
 * promotion-interval study. out is [rows, cols] F32 holding BF16 values.
 * Pinned by: brute force against exact rational sums on inputs whose every
 * partial sum is exactly representable (then QGMMA == exact dot), and the
 * reference's own case shape (rows 3, K 64, N 5, scales 5.75/3.25/0.03125). */
int oracle_qgmma_linear(const uint8_t *input_codes, const uint8_t *weight_codes,
                        size_t rows, size_t inner, size_t cols,
                        float output_scale, size_t group_k, float *out);

/* ---- F32 ops of src/cpu_reference.cpp (pinned by tests/vectors/cpu_ops.json
 * and the closed-form cases of tests/test_cpu_reference.cpp:154-250). */
int oracle_rms_norm(const float *x, size_t rows, size_t width,
                    const float *scale, float eps, float *out);
int oracle_linear_f32(const float *x, size_t rows, size_t in_features,
                      const float *weight, size_t out_features,
                      const float *bias, float *out);
int oracle_gated_mlp_f32(const float *x, size_t rows, size_t width,
                         size_t inner, const float *l1, const float *l2,
                         const float *l3, int gelu, float *out);
/* orientation 0 = cross-correlation, 1 = causal convolution;
 * bias_mode 0 = add, 1 = multiply-input (HCM's D*x). */
int oracle_causal_fir(const float *x, size_t length, size_t channels,
                      const float *weight, size_t kernel, const float *bias,
                      int orientation, int bias_mode, float *out);
int oracle_hcl_recurrence(const float *x2, const float *x1, const float *v,
                          size_t length, size_t width, const float *direct,
                          const float *log_poles, const float *residues,
                          size_t state_size, float *state, float *out);
int oracle_apply_rope(float *q, float *k, size_t length, size_t heads,
                      size_t head_dim, const float *inv_freq,
                      size_t position_offset, float position_scale);
int oracle_causal_attention(const float *q, const float *k, const float *v,
                            size_t length, size_t heads, size_t head_dim,
                            float *out);

/* ---- Model-path operators, following src/cpu/model.cpp exactly (BF16
 * weights read as raw bits, AVX2 8-lane FMA dot order :208-226).
 * linear: out[r,o] = dot(x[r,:], W[o,:]) (+ bf16 bias[o]). */
int oracle_linear_bf16w(const float *x, size_t rows, size_t in_features,
                        const uint16_t *weight, size_t out_features,
                        const uint16_t *bias, float *out, int threads);

/* Hyena mixer of one block (src/cpu/model.cpp:546-605) applied to an F32
 * projection P[L, 3W] (already projected), with zero initial caches.
 * kind: 0 = HCS, 1 = HCM, 2 = HCL. Weight arrays are F32 copies of the
 * artifact tensors: short_w [3W*short_len], inner_w [groups*inner_len]
 * (HCS/HCM), direct [W] (HCM/HCL), log_poles/residues [W*state] (HCL). */
int oracle_hyena_mixer(int kind, const float *projection, size_t length,
                       size_t width, const float *short_w, size_t short_len,
                       const float *inner_w, size_t groups, size_t inner_len,
                       const float *direct, const float *log_poles,
                       const float *residues, size_t state_size, float *out);

/* ---- Whole model (src/cpu/model.cpp:607-714 driven like the C ABI chunk
 * loop src/c_api.cpp:908-936). Reads an evo2-runtime-v1 Safetensors file.
 * Pinned by: bit-exact comparison with the reference libevo.so built from
 * /root/reference sources (oracle/_ref) on the same artifacts. */
void *oracle_model_load(const char *path, char *error, size_t error_size);
void oracle_model_free(void *model);
size_t oracle_model_width(const void *model);
size_t oracle_model_vocab(const void *model);
size_t oracle_model_layers(const void *model);
/* logits: [n, vocab]. chunk = tokens per forward (256 in the reference CPU
 * arena; results do not depend on it). capture_layer < layers additionally
 * copies that block's output hidden state [n, width] into capture. */
int oracle_model_prefill(void *model, const uint32_t *tokens, size_t n,
                         size_t chunk, float *logits, size_t capture_layer,
                         float *capture, int threads);
/* capture_layer == SIZE_MAX copies every block's output: capture holds
 * [layers][n][width]. */
/* Load-time FP8 conversion of the BF16 Hyena projections (the converter's
 * rule, evo.cpp tools/evo/checkpoint.py:393-396): weight_scale = 448 /
 * amax(W), codes = E4M3(W * weight_scale), input_scale = 448 / input_amax,
 * output_scale = 1 / (input_scale * weight_scale).
 * Pinned by: the same model written with codes and scales computed by the
 * artifact writer's independent numpy encoder (tests/test_oracle.py). */
int oracle_model_convert_fp8(void *model, float input_amax);
const char *oracle_last_error(void);
/* Design experiment (off by default): BF16-weight linears of the classes in
 * `mask` (bit 0 projections, 1 out-projection, 2 MLP l1/l2, 3 MLP l3) run as
 * hi . W + E4M3(lo) . E4M3(W) with E8M0 scales per 32 K; bit 4 rounds the
 * attention keys and bit 5 the values to BF16 (two-pass split products);
 * bit 6 makes hi FP16 instead of BF16, bit 7 drops the lo pass, bit 8 uses
 * one E4M3 scale per row instead of per 32-K block. Not a reference
 * function. */
void oracle_set_lo_emulation(unsigned mask);

#ifdef __cplusplus
}
#endif

#endif
