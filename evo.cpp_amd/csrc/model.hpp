// SPDX-License-Identifier: Apache-2.0
// HIP backend model (device-resident weights) and context (activation arena,
// continuation caches) for StripedHyena2 prefill on one MI355X.
//
// Mirrors the backend contract of evo.cpp's `cpu::Model` / `cpu::Context`
// (`include/evo/cpu/model.hpp:75-185`) and `cuda::PipelineModel`
// (`include/evo/cuda/model.hpp:107-227`): a model owns one copy of the
// weights; a context shares them and owns its arena, caches and stream;
// prefill / prefill_chunk / position / activation_capacity keep the same
// meaning.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "artifact.hpp"
#include "ops.hpp"
#include "status.hpp"

namespace evo::hip {

class DeviceBuffer {
public:
  DeviceBuffer() = default;
  ~DeviceBuffer() { reset(); }
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
  DeviceBuffer(DeviceBuffer &&other) noexcept { *this = std::move(other); }
  DeviceBuffer &operator=(DeviceBuffer &&other) noexcept {
    if (this != &other) {
      reset();
      ptr_ = other.ptr_;
      bytes_ = other.bytes_;
      other.ptr_ = nullptr;
      other.bytes_ = 0;
    }
    return *this;
  }
  Status allocate(size_t bytes, const char *what);
  Status upload(const void *host, size_t bytes, const char *what);
  void reset();
  template <typename T> T *as() const { return static_cast<T *>(ptr_); }
  size_t bytes() const { return bytes_; }

private:
  void *ptr_{nullptr};
  size_t bytes_{0};
};

enum class Mixer { kHcs, kHcm, kHcl, kAttention };

struct Layer {
  Mixer type{Mixer::kHcs};
  DeviceBuffer pre_norm, post_norm;        // F32 [W]
  DeviceBuffer projection;                 // BF16 [3W, W] or E4M3 [3W, W]
  bool fp8{false};
  float fp8_input_scale{0}, fp8_output_scale{0};
  DeviceBuffer out_weight, out_bias;       // BF16 [W, W], [W]
  DeviceBuffer out_weight16;               // FP16 copy of out_weight (W % 32 == 0)
  DeviceBuffer projection16;               // FP16 copy of an attention Wqkv
  DeviceBuffer short_filter;               // BF16 [3W, short_len]
  DeviceBuffer inner_filter;               // F32 [groups, len]
  DeviceBuffer direct;                     // F32 [W]
  DeviceBuffer poles, residues;            // F32 [W, S]
  DeviceBuffer inv_freq;                   // F32 [head_dim / 2]
  DeviceBuffer mlp_in;                     // BF16 [2*Fp, W], l1/l2 interleaved by 32 rows
  DeviceBuffer mlp_out;                    // BF16 [W, F]
};

struct ModelConfig {
  std::string model_id, architecture;
  size_t vocab{0}, width{0}, layers{0}, heads{0}, state{0}, inner{0},
      inner_padded{0}, short_len{0}, hcs_len{0}, hcm_len{0}, hcs_groups{0},
      hcm_groups{0}, max_seqlen{0};
  float eps{0}, rope_scale{0};
  bool column_split{false};
  size_t head_dim() const { return width / heads; }
};

class Model {
public:
  // fp8_projections converts BF16 Hyena input projections to software E4M3
  // at load (artifacts that already store F8_E4M3 keep their own scales).
  Status load(const Artifact &artifact, int device, bool allow_synthetic,
              bool fp8_projections);
  const ModelConfig &config() const { return config_; }
  int device() const { return device_; }

private:
  friend class Context;
  ModelConfig config_;
  int device_{0};
  DeviceBuffer embedding;   // BF16 [V, W] (also the tied unembedding)
  DeviceBuffer final_norm;  // F32 [W]
  std::vector<Layer> layer;
};

struct ContextOptions {
  bool split_activations{true};   // "hip-f32" (true) or "hip-bf16" (false)
  bool f16_proj{false};  // out- and attention projections on one FP16 pass ("+f16-proj")
  bool f16_out{false};   // out-projections only on one FP16 pass ("+f16-out")
  Fp8Mode fp8_mode{kFp8MfmaK128};
};

class Context {
public:
  Context() = default;
  ~Context();
  Status initialize(std::shared_ptr<const Model> model, size_t capacity,
                    const ContextOptions &options);
  // Runs rows tokens starting at position() (0 for the first chunk).
  // `logits` (host, [rows, vocab]) and/or `capture` (host, [rows, width] hidden
  // state after block capture_layer) receive the outputs.
  Status forward(const uint32_t *tokens, size_t rows, bool initial,
                 float *logits, size_t capture_layer, float *capture);
  // forward() with logits left in the context's pinned staging buffer:
  // *logits points at [rows, vocab] F32 there until the next call.
  Status forward_view(const uint32_t *tokens, size_t rows, bool initial,
                      const float **logits);
  // Whole-sequence prefill with tokens and logits ([count, vocab] F32) in
  // device memory: chunks are enqueued back to back on the context stream,
  // one synchronisation at the end, no host transfer of activations.
  Status prefill_resident(const uint32_t *device_tokens, size_t count,
                          float *device_logits);
  // HIP events around each layer's MLP l1/l2 product (off by default), for
  // timing the dominant kernel inside real prefills; product_time reads the
  // launches of the last enqueued chunk (the caller has synchronised). A
  // decode step is a chunk too and replaces them; (0, 0) before any chunk
  // and after a chunk that failed before its first product.
  Status set_product_timing(bool on);
  Status product_time(float *ms, size_t *launches) const;
  size_t position() const { return position_; }
  size_t activation_capacity() const { return arena_rows_; }
  size_t capacity() const { return capacity_; }
  const ModelConfig &config() const { return model_->config(); }
  const char *profile() const { return profile_.c_str(); }
  hipStream_t stream() const { return stream_; }

private:
  Status enqueue(const uint32_t *device_tokens, size_t rows, bool initial,
                 float *device_logits, size_t capture_layer, float *capture);
  Status finish();
  Status run_layers(size_t rows, size_t capture_layer, float *capture);
  void reset_caches();
  // workspace_ holds pending_'s partials until the next norm of hidden_
  // consumes them: every other user of workspace_ checks this first.
  Status workspace_free(const char *user) const;

  std::shared_ptr<const Model> model_;
  // Split-K partials of the last MLP l3 product not yet summed into hidden_
  // (short chunks): the next RMSNorm of hidden_ sums them as it reads them.
  SplitPartials pending_{};
  std::vector<hipEvent_t> timing_events_;  // start / stop per layer, or empty
  size_t timed_pairs_{0};  // event pairs the last enqueued chunk recorded
  unsigned hi_only_{0};    // diagnostic: GEMM classes run on the hi plane only
  ContextOptions options_;
  std::string profile_;
  hipStream_t stream_{nullptr};
  size_t capacity_{0}, cache_capacity_{0}, arena_rows_{0}, position_{0};
  bool valid_{false};
  DeviceBuffer tokens_, hidden_, residual_, normed_, projected_, mixed_, query_,
      gated_, logits_, codes_, workspace_, flag_;
  size_t workspace_bytes_{0};
  struct Cache {
    DeviceBuffer short_history, inner_history, modal_state, keys, values;
  };
  std::vector<Cache> cache_;
  // Device table of the Hyena caches (ZeroRegion entries) that reset_caches
  // clears in one launch.
  DeviceBuffer reset_table_;
  size_t reset_count_{0}, reset_max_words_{0};
  float *host_logits_{nullptr};
  int *host_flag_{nullptr};
};

}  // namespace evo::hip
