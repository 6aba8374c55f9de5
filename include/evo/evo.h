/* SPDX-License-Identifier: Apache-2.0
 *
 * evo C ABI as exported by libevo_hip.so, the MI355X (gfx950) StripedHyena2
 * prefill library.
 *
 * Drop-in surface: every declaration below has the name, argument meaning,
 * ownership rule and status codes of evo.cpp's `include/evo/evo.h:133-210`
 * (ABI 1.5.0). Additions, kept ABI-compatible as a minor bump (1.6.0):
 *   - EVO_BACKEND_HIP = 4  (beside EVO_BACKEND_{AUTO,CUDA,CPU,MPS},
 *     reference `include/evo/evo.h:45-50`);
 *   - EVO_STATUS_HIP = 8   (style of EVO_STATUS_CUDA/MPS, reference :34-43);
 *   - context flags selecting the HIP numeric profile.
 * EVO_BACKEND_AUTO resolves to HIP in this library. CPU/CUDA/MPS requests
 * return EVO_STATUS_UNSUPPORTED: this library implements the HIP backend only.
 */
#ifndef EVO_EVO_H
#define EVO_EVO_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define EVO_API __attribute__((visibility("default")))
#else
#define EVO_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define EVO_ABI_VERSION_MAJOR 1u
#define EVO_ABI_VERSION_MINOR 6u
#define EVO_ABI_VERSION_PATCH 0u
#define EVO_ABI_VERSION_ENCODE(major, minor, patch)                            \
  ((((uint32_t)(major) & 0xffu) << 24u) |                                      \
   (((uint32_t)(minor) & 0xffu) << 16u) | ((uint32_t)(patch) & 0xffffu))
#define EVO_ABI_VERSION_CURRENT                                                \
  EVO_ABI_VERSION_ENCODE(EVO_ABI_VERSION_MAJOR, EVO_ABI_VERSION_MINOR,         \
                         EVO_ABI_VERSION_PATCH)

/* Reference: include/evo/evo.h:34-43, plus EVO_STATUS_HIP. */
typedef enum evo_status {
  EVO_STATUS_OK = 0,
  EVO_STATUS_INVALID_ARGUMENT = 2,
  EVO_STATUS_IO = 3,
  EVO_STATUS_MODEL_FORMAT = 4,
  EVO_STATUS_UNSUPPORTED = 5,
  EVO_STATUS_CUDA = 6,
  EVO_STATUS_MPS = 7,
  EVO_STATUS_HIP = 8,
  EVO_STATUS_INTERNAL = 70
} evo_status;

/* Reference: include/evo/evo.h:45-50, plus EVO_BACKEND_HIP. */
typedef enum evo_backend {
  EVO_BACKEND_AUTO = 0,
  EVO_BACKEND_CUDA = 1,
  EVO_BACKEND_CPU = 2,
  EVO_BACKEND_MPS = 3,
  EVO_BACKEND_HIP = 4
} evo_backend;

enum {
  /* Reference: include/evo/evo.h:52-56. */
  EVO_MODEL_FLAG_TEST_ONLY_ALLOW_SYNTHETIC = 1u << 0u,
  /* HIP: convert BF16 Hyena input projections to software E4M3 at load with
   * the converter's per-tensor amax rule (weight scale 448/amax(W), fixed
   * activation scale 448/8). Artifacts storing F8_E4M3 keep their scales. */
  EVO_MODEL_FLAG_HIP_FP8_PROJECTIONS = 1u << 8u
};

enum {
  /* Reference: include/evo/evo.h:58-62. Accepted for ABI compatibility; the
   * HIP backend keeps every K/V row resident (288 GB HBM) and rejects it. */
  EVO_CONTEXT_FLAG_FAST_Q8_KV = 1u << 0u,
  /* HIP numeric profile "hip-bf16": GEMM activations rounded to BF16 (one
   * MFMA pass) instead of the default "hip-f32" profile, whose GEMMs split
   * each F32 activation into two BF16 terms. */
  EVO_CONTEXT_FLAG_HIP_BF16 = 1u << 8u,
  /* Software-FP8 projections run through the bit-exact integer QGMMA
   * emulation ("+fp8-exact") instead of the default E4M3 MFMA path, which
   * promotes each 128-K chunk into an E8M13-truncated accumulator. */
  EVO_CONTEXT_FLAG_HIP_FP8_EXACT = 1u << 9u,
  /* E4M3 MFMA path promoting every 32-K chunk (the reference's QGMMA group
   * size) instead of every 128 K ("+fp8-k32"); exclusive with FP8_EXACT. */
  EVO_CONTEXT_FLAG_HIP_FP8_K32 = 1u << 10u,
  /* "+f16-proj": the out-projections (mixer output times out_proj /
   * out_filter_dense) and the attention input projections (Wqkv) run as one
   * FP16 MFMA pass (activation rounded to FP16, weight converted to FP16 at
   * load) instead of two split-BF16 passes. The MLP products and the FP8
   * Hyena projections are unchanged. */
  EVO_CONTEXT_FLAG_HIP_F16_PROJ = 1u << 11u,
  /* "+f16-out": only the out-projections run as one FP16 MFMA pass (the
   * attention input projections stay split BF16); implied by F16_PROJ. With
   * either flag, a prefill whose FP16 activations leave the FP16 range
   * (+-65504) or hold NaN fails with EVO_STATUS_UNSUPPORTED. */
  EVO_CONTEXT_FLAG_HIP_F16_OUT = 1u << 12u
};

typedef struct evo_model evo_model;
typedef struct evo_context evo_context;
typedef struct evo_batch evo_batch;
typedef struct evo_sampler evo_sampler;

/* Reference: include/evo/evo.h:69-75. */
typedef struct evo_model_params {
  size_t struct_size;
  evo_backend backend;
  const int32_t *devices;
  size_t device_count;
  uint32_t flags;
} evo_model_params;

/* Reference: include/evo/evo.h:77-81. */
typedef struct evo_context_params {
  size_t struct_size;
  size_t context_size;
  uint32_t flags;
} evo_context_params;

/* Reference: include/evo/evo.h:83-89. */
typedef struct evo_sampler_params {
  size_t struct_size;
  float temperature;
  size_t top_k;
  float top_p;
  uint64_t seed;
} evo_sampler_params;

/* Reference: include/evo/evo.h:94-99. */
typedef struct evo_embedding_options {
  size_t struct_size;
  const char *preset;
  size_t layer;
  const char *pooling;
} evo_embedding_options;

/* Reference: include/evo/evo.h:103-118. */
typedef struct evo_embedding_result_info {
  size_t struct_size;
  const char *resolved_preset;
  const char *hidden_tap;
  const char *pooling;
  size_t layer;
  size_t original_length;
  size_t effective_length;
  size_t crop_left;
  size_t crop_right;
  size_t pad_left;
  size_t pad_right;
  size_t token_count;
  size_t rows;
  size_t columns;
} evo_embedding_result_info;

/* Reference: include/evo/evo.h:122-131. The logits view is valid only for
 * the duration of the callback; a non-OK return aborts the call and
 * permanently invalidates the context. */
typedef evo_status (*evo_logits_callback)(const float *logits, size_t rows,
                                          size_t columns, size_t token_offset,
                                          void *user_data);
typedef evo_status (*evo_embedding_callback)(const float *embedding,
                                             size_t rows, size_t columns,
                                             size_t token_offset,
                                             void *user_data);
typedef evo_status (*evo_embedding_ex_callback)(
    const float *embedding, size_t rows, size_t columns, size_t token_offset,
    const evo_embedding_result_info *info, void *user_data);

/* Reference: include/evo/evo.h:133-210 (same names and contracts). */
EVO_API uint32_t evo_abi_version(void);
EVO_API const char *evo_version_string(void);
EVO_API const char *evo_status_name(evo_status status);
EVO_API const char *evo_backend_name(evo_backend backend);
EVO_API const char *evo_last_error(void);

EVO_API evo_model_params evo_model_default_params(void);
EVO_API evo_context_params evo_context_default_params(void);
EVO_API evo_sampler_params evo_sampler_default_params(void);
EVO_API evo_embedding_options evo_embedding_default_options(void);

EVO_API evo_status evo_model_load(const char *path,
                                  const evo_model_params *params,
                                  evo_model **model_out);
EVO_API void evo_model_free(evo_model *model);
EVO_API evo_backend evo_model_backend(const evo_model *model);
EVO_API const char *evo_model_id(const evo_model *model);
EVO_API const char *evo_model_architecture(const evo_model *model);
EVO_API const char *evo_model_profile(const evo_model *model);
EVO_API size_t evo_model_vocab_size(const evo_model *model);
EVO_API size_t evo_model_max_context(const evo_model *model);
EVO_API size_t evo_model_embedding_width(const evo_model *model);
EVO_API size_t evo_model_layer_count(const evo_model *model);
EVO_API evo_status evo_model_encode(const evo_model *model,
                                    const uint8_t *sequence,
                                    size_t sequence_length, uint32_t *tokens,
                                    size_t token_capacity,
                                    size_t *token_count);
EVO_API evo_status evo_model_decode_token(const evo_model *model,
                                          uint32_t token, uint8_t *byte_out);

EVO_API evo_status evo_context_create(const evo_model *model,
                                      const evo_context_params *params,
                                      evo_context **context_out);
EVO_API void evo_context_free(evo_context *context);
EVO_API size_t evo_context_position(const evo_context *context);
EVO_API size_t evo_context_capacity(const evo_context *context);
EVO_API const char *evo_context_profile(const evo_context *context);
EVO_API evo_status evo_context_prefill(evo_context *context,
                                       const evo_batch *batch,
                                       evo_logits_callback callback,
                                       void *user_data);
/* One cached decode step after a prefill: the token at position
 * evo_context_position() advances every cache and its [1, vocab] logits go
 * to the callback (reference `include/evo/evo.h:183-186`). */
EVO_API evo_status evo_context_decode(evo_context *context, uint32_t token,
                                      evo_logits_callback callback,
                                      void *user_data);
/* Hidden-state capture after block `layer` (layer == layer_count selects the
 * final-norm output), streamed per prefill chunk like the logits. */
EVO_API evo_status evo_context_embed(evo_context *context,
                                     const evo_batch *batch, size_t layer,
                                     evo_embedding_callback callback,
                                     void *user_data);
EVO_API evo_status evo_context_embed_ex(evo_context *context,
                                        const evo_batch *batch,
                                        const evo_embedding_options *options,
                                        evo_embedding_ex_callback callback,
                                        void *user_data);

EVO_API evo_status evo_batch_create(size_t sequence_capacity,
                                    evo_batch **batch_out);
EVO_API void evo_batch_free(evo_batch *batch);
EVO_API void evo_batch_clear(evo_batch *batch);
EVO_API evo_status evo_batch_add_sequence(evo_batch *batch,
                                          const uint8_t *sequence,
                                          size_t sequence_length);
EVO_API size_t evo_batch_sequence_count(const evo_batch *batch);
EVO_API size_t evo_batch_token_count(const evo_batch *batch);

EVO_API evo_status evo_sampler_create(const evo_sampler_params *params,
                                      evo_sampler **sampler_out);
EVO_API void evo_sampler_free(evo_sampler *sampler);
EVO_API evo_status evo_sampler_sample(evo_sampler *sampler, const float *logits,
                                      size_t logits_count, uint32_t *token_out);

#ifdef __cplusplus
}
#endif

#endif
