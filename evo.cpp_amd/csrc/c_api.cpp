// SPDX-License-Identifier: Apache-2.0
// evo C ABI (include/evo/evo.h) over the HIP backend, and the operator-level
// ABI (include/evo/hip_ops.h).
//
// Conventions follow evo.cpp `src/c_api.cpp`: thread-local last error
// (:40-72), no exception crosses the boundary (`protect`, :74-85), parameter
// structs start with struct_size, batch size exactly one, fresh context per
// prefill, chunk loop over the activation arena with a logits callback per
// chunk (:908-936), and a context poisoned by any failure after its state
// started to advance (:904-907).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <exception>
#include <functional>
#include <limits>
#include <memory>
#include <mutex>
#include <new>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#include "artifact.hpp"
#include "evo/evo.h"
#include "evo/hip_ops.h"
#include "model.hpp"
#include "ops.hpp"

namespace {

thread_local std::string last_error;

evo_status publish(const evo::Status &status) {
  if (status.ok()) {
    last_error.clear();
    return EVO_STATUS_OK;
  }
  const std::string prefix = std::string(evo::error_code_name(status.code())) + ":";
  last_error = status.message().rfind(prefix, 0) == 0
                   ? status.message()
                   : std::string(evo::error_code_name(status.code())) + ": " + status.message();
  return static_cast<evo_status>(status.code());
}

evo_status publish(evo_status status, std::string message) {
  if (status == EVO_STATUS_OK)
    last_error.clear();
  else
    last_error = std::move(message);
  return status;
}

template <typename F> evo_status protect(F &&function) noexcept {
  try {
    return function();
  } catch (const std::bad_alloc &) {
    return publish(EVO_STATUS_INTERNAL, "internal: allocation failed");
  } catch (const std::exception &error) {
    return publish(EVO_STATUS_INTERNAL,
                   std::string("internal: unexpected exception: ") + error.what());
  } catch (...) {
    return publish(EVO_STATUS_INTERNAL, "internal: unknown exception");
  }
}

bool valid_status(const evo_status s) {
  return s == EVO_STATUS_OK || s == EVO_STATUS_INVALID_ARGUMENT || s == EVO_STATUS_IO ||
         s == EVO_STATUS_MODEL_FORMAT || s == EVO_STATUS_UNSUPPORTED ||
         s == EVO_STATUS_CUDA || s == EVO_STATUS_MPS || s == EVO_STATUS_HIP ||
         s == EVO_STATUS_INTERNAL;
}

struct ModelState {
  evo::Artifact artifact;
  std::shared_ptr<evo::hip::Model> weights;
  std::string model_id, architecture, profile;
  int device{0};
};

}  // namespace

struct evo_model {
  std::shared_ptr<ModelState> state;
};

struct evo_context {
  std::shared_ptr<ModelState> state;
  std::unique_ptr<evo::hip::Context> hip;
  bool failed{false};
};

struct evo_batch {
  size_t capacity{0};
  size_t tokens{0};
  std::vector<std::vector<uint8_t>> sequences;
};

struct evo_sampler {
  evo_sampler_params params;
  std::mt19937_64 random;
};

namespace {

using ChunkSink = std::function<evo_status(const float *, size_t, size_t, size_t)>;

// Shared chunk loop of prefill and embed (`src/c_api.cpp:862-998`).
evo_status run_prefill(evo_context *context, const evo_batch *batch,
                       size_t capture_layer, const ChunkSink &sink) {
  if (context->failed)
    return publish(EVO_STATUS_INVALID_ARGUMENT,
                   "invalid_argument: context is invalid after a prior failure");
  if (batch->sequences.size() != 1)
    return publish(EVO_STATUS_UNSUPPORTED,
                   "unsupported: exact backend currently requires batch size one");
  const auto &sequence = batch->sequences.front();
  if (sequence.empty() || context->hip->position() != 0)
    return publish(EVO_STATUS_INVALID_ARGUMENT,
                   "invalid_argument: prefill requires a fresh context and a "
                   "nonempty sequence within capacity");
  // Byte-identity tokenizer (`src/tokenizer.cpp:24-33`).
  std::vector<uint32_t> tokens(sequence.begin(), sequence.end());
  if (tokens.size() > context->hip->capacity())
    return publish(EVO_STATUS_INVALID_ARGUMENT,
                   "invalid_argument: encoded sequence exceeds context capacity");
  context->failed = true;
  const auto &config = context->hip->config();
  const size_t chunk = context->hip->activation_capacity();
  const bool capture = capture_layer != std::numeric_limits<size_t>::max();
  const size_t columns = capture ? config.width : config.vocab;
  // Logits are handed to the callback straight from the context's pinned
  // staging buffer; captured hidden states go through a host vector.
  std::vector<float> captured(capture ? std::min(chunk, tokens.size()) * columns : 0);
  size_t offset = 0;
  while (offset < tokens.size()) {
    const size_t rows = std::min(chunk, tokens.size() - offset);
    const float *values = captured.data();
    const auto status =
        capture ? context->hip->forward(tokens.data() + offset, rows, offset == 0, nullptr,
                                        capture_layer, captured.data())
                : context->hip->forward_view(tokens.data() + offset, rows, offset == 0,
                                             &values);
    if (!status.ok())
      return publish(status);
    const evo_status callback = sink(values, rows, columns, offset);
    if (callback != EVO_STATUS_OK)
      return publish(valid_status(callback) ? callback : EVO_STATUS_INTERNAL,
                     "callback: consumer aborted HIP prefill");
    offset += rows;
  }
  context->failed = false;
  return publish(evo::Status::Ok());
}

}  // namespace

extern "C" {

uint32_t evo_abi_version(void) { return EVO_ABI_VERSION_CURRENT; }
const char *evo_version_string(void) { return "0.1.0-hip"; }

const char *evo_status_name(evo_status status) {
  if (!valid_status(status))
    return "unknown";
  return evo::error_code_name(static_cast<evo::ErrorCode>(status));
}

const char *evo_backend_name(evo_backend backend) {
  switch (backend) {
  case EVO_BACKEND_AUTO: return "auto";
  case EVO_BACKEND_CUDA: return "cuda";
  case EVO_BACKEND_CPU: return "cpu";
  case EVO_BACKEND_MPS: return "mps";
  case EVO_BACKEND_HIP: return "hip";
  }
  return "unknown";
}

const char *evo_last_error(void) { return last_error.c_str(); }

evo_model_params evo_model_default_params(void) {
  return {sizeof(evo_model_params), EVO_BACKEND_AUTO, nullptr, 0, 0};
}
evo_context_params evo_context_default_params(void) {
  return {sizeof(evo_context_params), 4096, 0};
}
evo_sampler_params evo_sampler_default_params(void) {
  return {sizeof(evo_sampler_params), 1.0F, 1, 1.0F, 0};
}
evo_embedding_options evo_embedding_default_options(void) {
  return {sizeof(evo_embedding_options), nullptr,
          std::numeric_limits<size_t>::max(), nullptr};
}

evo_status evo_model_load(const char *path, const evo_model_params *params,
                          evo_model **model_out) {
  if (model_out != nullptr)
    *model_out = nullptr;
  return protect([&]() -> evo_status {
    if (path == nullptr || path[0] == '\0' || model_out == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: model path/output is null or empty");
    if (params != nullptr && params->struct_size < sizeof(evo_model_params))
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: evo_model_params is too small");
    const evo_model_params options = params == nullptr ? evo_model_default_params() : *params;
    if (options.backend != EVO_BACKEND_AUTO && options.backend != EVO_BACKEND_HIP &&
        options.backend != EVO_BACKEND_CPU && options.backend != EVO_BACKEND_CUDA &&
        options.backend != EVO_BACKEND_MPS)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: unknown model backend");
    if (options.backend != EVO_BACKEND_AUTO && options.backend != EVO_BACKEND_HIP)
      return publish(EVO_STATUS_UNSUPPORTED,
                     "unsupported: this evo library implements the HIP backend only");
    const uint32_t known_flags = EVO_MODEL_FLAG_TEST_ONLY_ALLOW_SYNTHETIC |
                                 EVO_MODEL_FLAG_HIP_FP8_PROJECTIONS;
    if ((options.flags & ~known_flags) != 0 ||
        options.device_count > 1 || (options.device_count != 0 && options.devices == nullptr))
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: invalid model flags/device list (one device)");
    auto state = std::make_shared<ModelState>();
    state->device = options.device_count == 0 ? 0 : options.devices[0];
    if (state->device < 0)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: device must be nonnegative");
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices <= state->device)
      return publish(EVO_STATUS_HIP, "hip: no usable HIP device");
    auto status = state->artifact.open(path);
    if (!status.ok())
      return publish(status);
    std::string abi;
    if (state->artifact.profile() != "evo2-runtime-v1" ||
        !state->artifact.meta_string("runtime.abi", &abi).ok() ||
        abi != "evo2-safetensors-v1")
      return publish(EVO_STATUS_UNSUPPORTED,
                     "unsupported: artifact architecture/profile/ABI is not registered");
    state->weights = std::make_shared<evo::hip::Model>();
    status = state->weights->load(state->artifact, state->device,
                                  (options.flags & EVO_MODEL_FLAG_TEST_ONLY_ALLOW_SYNTHETIC) != 0,
                                  (options.flags & EVO_MODEL_FLAG_HIP_FP8_PROJECTIONS) != 0);
    if (!status.ok())
      return publish(status);
    state->model_id = state->weights->config().model_id;
    state->architecture = state->weights->config().architecture;
    state->profile = state->artifact.profile();
    *model_out = new evo_model{std::move(state)};
    return publish(evo::Status::Ok());
  });
}

void evo_model_free(evo_model *model) { delete model; }

evo_backend evo_model_backend(const evo_model *model) {
  return model == nullptr ? EVO_BACKEND_AUTO : EVO_BACKEND_HIP;
}
const char *evo_model_id(const evo_model *m) {
  return m == nullptr ? "" : m->state->model_id.c_str();
}
const char *evo_model_architecture(const evo_model *m) {
  return m == nullptr ? "" : m->state->architecture.c_str();
}
const char *evo_model_profile(const evo_model *m) {
  return m == nullptr ? "" : m->state->profile.c_str();
}
size_t evo_model_vocab_size(const evo_model *m) {
  return m == nullptr ? 0 : m->state->weights->config().vocab;
}
size_t evo_model_max_context(const evo_model *m) {
  return m == nullptr ? 0 : m->state->weights->config().max_seqlen;
}
size_t evo_model_embedding_width(const evo_model *m) {
  return m == nullptr ? 0 : m->state->weights->config().width;
}
size_t evo_model_layer_count(const evo_model *m) {
  return m == nullptr ? 0 : m->state->weights->config().layers;
}

evo_status evo_model_encode(const evo_model *model, const uint8_t *sequence,
                            size_t length, uint32_t *tokens, size_t capacity,
                            size_t *count) {
  return protect([&]() -> evo_status {
    if (model == nullptr || count == nullptr || (sequence == nullptr && length != 0))
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: model encoder arguments are invalid");
    *count = length;
    if (tokens == nullptr)
      return publish(evo::Status::Ok());
    if (capacity < length)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: token buffer is too small");
    for (size_t i = 0; i < length; ++i)
      tokens[i] = sequence[i];
    return publish(evo::Status::Ok());
  });
}

evo_status evo_model_decode_token(const evo_model *model, uint32_t token,
                                  uint8_t *byte_out) {
  return protect([&]() -> evo_status {
    if (model == nullptr || byte_out == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: model detokenizer arguments are invalid");
    if (token > 255)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: token " + std::to_string(token) +
                         " has no byte representation");
    *byte_out = static_cast<uint8_t>(token);
    return publish(evo::Status::Ok());
  });
}

evo_status evo_context_create(const evo_model *model, const evo_context_params *params,
                              evo_context **context_out) {
  if (context_out != nullptr)
    *context_out = nullptr;
  return protect([&]() -> evo_status {
    if (model == nullptr || !model->state || context_out == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: model/context output is null");
    if (params != nullptr && params->struct_size < sizeof(evo_context_params))
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: evo_context_params is too small");
    const evo_context_params options = params == nullptr ? evo_context_default_params() : *params;
    const uint32_t known = EVO_CONTEXT_FLAG_HIP_BF16 | EVO_CONTEXT_FLAG_HIP_FP8_EXACT |
                           EVO_CONTEXT_FLAG_HIP_FP8_K32 | EVO_CONTEXT_FLAG_HIP_F16_PROJ |
                           EVO_CONTEXT_FLAG_HIP_F16_OUT;
    const uint32_t fp8_modes = EVO_CONTEXT_FLAG_HIP_FP8_EXACT | EVO_CONTEXT_FLAG_HIP_FP8_K32;
    if (options.context_size == 0 || (options.flags & ~known) != 0 ||
        (options.flags & fp8_modes) == fp8_modes)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: invalid context parameters");
    const auto &config = model->state->weights->config();
    if (options.context_size > config.max_seqlen)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: requested context exceeds model maximum");
    evo::hip::ContextOptions hip_options;
    hip_options.split_activations = (options.flags & EVO_CONTEXT_FLAG_HIP_BF16) == 0;
    hip_options.f16_proj = (options.flags & EVO_CONTEXT_FLAG_HIP_F16_PROJ) != 0;
    hip_options.f16_out = (options.flags & EVO_CONTEXT_FLAG_HIP_F16_OUT) != 0;
    hip_options.fp8_mode = (options.flags & EVO_CONTEXT_FLAG_HIP_FP8_EXACT) != 0
                               ? evo::hip::kFp8Exact
                           : (options.flags & EVO_CONTEXT_FLAG_HIP_FP8_K32) != 0
                               ? evo::hip::kFp8MfmaK32
                               : evo::hip::kFp8MfmaK128;
    auto handle = std::make_unique<evo_context>();
    handle->state = model->state;
    handle->hip = std::make_unique<evo::hip::Context>();
    const auto status = handle->hip->initialize(model->state->weights,
                                                options.context_size, hip_options);
    if (!status.ok())
      return publish(status);
    *context_out = handle.release();
    return publish(evo::Status::Ok());
  });
}

void evo_context_free(evo_context *context) { delete context; }

size_t evo_context_position(const evo_context *context) {
  return context == nullptr || !context->hip ? 0 : context->hip->position();
}
size_t evo_context_capacity(const evo_context *context) {
  return context == nullptr || !context->hip ? 0 : context->hip->capacity();
}
const char *evo_context_profile(const evo_context *context) {
  return context == nullptr || !context->hip ? "" : context->hip->profile();
}

evo_status evo_context_prefill(evo_context *context, const evo_batch *batch,
                               evo_logits_callback callback, void *user_data) {
  return protect([&]() -> evo_status {
    if (context == nullptr || batch == nullptr || callback == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: prefill argument is null");
    return run_prefill(context, batch, std::numeric_limits<size_t>::max(),
                       [&](const float *v, size_t rows, size_t cols, size_t offset) {
                         return callback(v, rows, cols, offset, user_data);
                       });
  });
}

// One cached step: the token at position `offset` runs through every block
// as a one-row continuation (FIR histories, HCL modal state and K/V caches
// advance), and its logits go to the callback (`src/c_api.cpp:1000-1082`,
// StripedHyena2 decode = forward({token}) on the caches,
// `src/cpu/model.cpp:3475-3483`).
evo_status evo_context_decode(evo_context *context, uint32_t token,
                              evo_logits_callback callback, void *user_data) {
  return protect([&]() -> evo_status {
    if (context == nullptr || callback == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: decode argument is null");
    if (context->failed)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: context is invalid after a prior failure");
    const size_t offset = context->hip->position();
    const auto &config = context->hip->config();
    if (offset == 0 || offset >= context->hip->capacity() || token >= config.vocab)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: decode token/context is invalid");
    context->failed = true;
    std::vector<float> logits(config.vocab);
    const auto status = context->hip->forward(&token, 1, false, logits.data(),
                                              std::numeric_limits<size_t>::max(), nullptr);
    if (!status.ok())
      return publish(status);
    const evo_status callback_status = callback(logits.data(), 1, config.vocab, offset,
                                                user_data);
    if (callback_status != EVO_STATUS_OK)
      return publish(valid_status(callback_status) ? callback_status : EVO_STATUS_INTERNAL,
                     "callback: logits consumer aborted HIP decode");
    context->failed = false;
    return publish(evo::Status::Ok());
  });
}

evo_status evo_context_embed(evo_context *context, const evo_batch *batch, size_t layer,
                             evo_embedding_callback callback, void *user_data) {
  return protect([&]() -> evo_status {
    if (context == nullptr || batch == nullptr || callback == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: embed argument is null");
    if (layer >= context->hip->config().layers)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: embedding layer is outside the model");
    return run_prefill(context, batch, layer,
                       [&](const float *v, size_t rows, size_t cols, size_t offset) {
                         return callback(v, rows, cols, offset, user_data);
                       });
  });
}

evo_status evo_context_embed_ex(evo_context *context, const evo_batch *, const
                                evo_embedding_options *, evo_embedding_ex_callback, void *) {
  return protect([&]() -> evo_status {
    if (context == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: embed argument is null");
    return publish(EVO_STATUS_UNSUPPORTED,
                   "unsupported: embedding presets are not part of the HIP prefill library");
  });
}

evo_status evo_batch_create(size_t capacity, evo_batch **batch_out) {
  if (batch_out != nullptr)
    *batch_out = nullptr;
  return protect([&]() -> evo_status {
    if (batch_out == nullptr || capacity == 0)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: invalid batch capacity");
    auto batch = std::make_unique<evo_batch>();
    batch->capacity = capacity;
    *batch_out = batch.release();
    return publish(evo::Status::Ok());
  });
}

void evo_batch_free(evo_batch *batch) { delete batch; }

void evo_batch_clear(evo_batch *batch) {
  if (batch != nullptr) {
    batch->sequences.clear();
    batch->tokens = 0;
  }
}

evo_status evo_batch_add_sequence(evo_batch *batch, const uint8_t *sequence, size_t length) {
  return protect([&]() -> evo_status {
    if (batch == nullptr || (sequence == nullptr && length != 0))
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: invalid batch sequence");
    if (batch->sequences.size() >= batch->capacity)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: batch is full");
    batch->sequences.emplace_back(sequence, sequence + length);
    batch->tokens += length;
    return publish(evo::Status::Ok());
  });
}

size_t evo_batch_sequence_count(const evo_batch *batch) {
  return batch == nullptr ? 0 : batch->sequences.size();
}
size_t evo_batch_token_count(const evo_batch *batch) {
  return batch == nullptr ? 0 : batch->tokens;
}

// Sampler: evo.cpp `src/sampler.cpp:12-104` -- stable descending order (ties by
// lower index), top-k, temperature softmax in F64 relative to the top logit,
// nucleus cut, one mt19937_64 draw mapped to 53 bits.
evo_status evo_sampler_create(const evo_sampler_params *params, evo_sampler **out) {
  if (out != nullptr)
    *out = nullptr;
  return protect([&]() -> evo_status {
    if (out == nullptr || (params != nullptr && params->struct_size < sizeof(evo_sampler_params)))
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: invalid sampler params");
    const evo_sampler_params p = params == nullptr ? evo_sampler_default_params() : *params;
    if (!std::isfinite(p.temperature) || p.temperature <= 0.0F || !std::isfinite(p.top_p) ||
        p.top_p <= 0.0F || p.top_p > 1.0F ||
        p.top_k > static_cast<size_t>(std::numeric_limits<uint32_t>::max()) + 1)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: invalid sampling config");
    *out = new evo_sampler{p, std::mt19937_64(p.seed)};
    return publish(evo::Status::Ok());
  });
}

void evo_sampler_free(evo_sampler *sampler) { delete sampler; }

evo_status evo_sampler_sample(evo_sampler *sampler, const float *logits, size_t count,
                              uint32_t *token_out) {
  return protect([&]() -> evo_status {
    if (sampler == nullptr || logits == nullptr || token_out == nullptr || count == 0 ||
        count > static_cast<size_t>(std::numeric_limits<uint32_t>::max()) + 1)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: invalid sampler call");
    const auto &p = sampler->params;
    if (p.top_k > count)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: top-k exceeds the model vocabulary");
    for (size_t i = 0; i < count; ++i)
      if (!std::isfinite(logits[i]))
        return publish(EVO_STATUS_INVALID_ARGUMENT,
                       "invalid_argument: logit " + std::to_string(i) + " is not finite");
    std::vector<size_t> order(count);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
      if (logits[a] == logits[b])
        return a < b;
      return logits[a] > logits[b];
    });
    if (p.top_k == 1) {
      *token_out = static_cast<uint32_t>(order.front());
      return publish(evo::Status::Ok());
    }
    if (p.top_k != 0 && order.size() > p.top_k)
      order.resize(p.top_k);
    std::vector<double> weights;
    weights.reserve(order.size());
    const double top = static_cast<double>(logits[order.front()]) / p.temperature;
    double total = 0.0;
    for (size_t index : order) {
      const double w = std::exp(static_cast<double>(logits[index]) / p.temperature - top);
      weights.push_back(w);
      total += w;
    }
    if (p.top_p < 1.0F) {
      double cumulative = 0.0;
      size_t keep = 0;
      while (keep < weights.size() && cumulative / total < static_cast<double>(p.top_p)) {
        cumulative += weights[keep];
        ++keep;
      }
      order.resize(keep);
      weights.resize(keep);
      total = cumulative;
    }
    const double draw =
        static_cast<double>(sampler->random() >> 11U) * (1.0 / 9007199254740992.0) * total;
    double cumulative = 0.0;
    for (size_t i = 0; i < order.size(); ++i) {
      cumulative += weights[i];
      if (draw < cumulative || i + 1 == order.size()) {
        *token_out = static_cast<uint32_t>(order[i]);
        return publish(evo::Status::Ok());
      }
    }
    return publish(EVO_STATUS_INTERNAL, "internal: sampler failed to select a token");
  });
}

// ------------------------------------------------------------ operator ABI
evo_status evo_hip_context_prefill_resident(evo_context *context, const uint32_t *tokens,
                                            size_t count, float *logits) {
  return protect([&]() -> evo_status {
    if (context == nullptr || !context->hip)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: context is null");
    if (context->failed)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: context is invalid after a prior failure");
    context->failed = true;
    const auto status = context->hip->prefill_resident(tokens, count, logits);
    if (!status.ok())
      return publish(status);
    context->failed = false;
    return publish(evo::Status::Ok());
  });
}

evo_status evo_hip_context_set_product_timing(evo_context *context, int enable) {
  return protect([&]() -> evo_status {
    if (context == nullptr || !context->hip)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: context is null");
    return publish(context->hip->set_product_timing(enable != 0));
  });
}

evo_status evo_hip_context_product_time(const evo_context *context, float *ms,
                                        size_t *launches) {
  return protect([&]() -> evo_status {
    if (context == nullptr || !context->hip)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: context is null");
    return publish(context->hip->product_time(ms, launches));
  });
}

void *evo_hip_context_stream(const evo_context *context) {
  return context == nullptr || !context->hip ? nullptr : context->hip->stream();
}

size_t evo_hip_hyena_workspace_bytes(evo_hip_hyena_kind kind, size_t length, size_t width,
                                     size_t state_size) {
  return evo::hip::hyena_workspace_bytes(static_cast<int>(kind), length, width, state_size);
}

namespace {
// Typed dispatch shared by the workspace and the static-scratch entry points.
evo::Status hyena_dispatch(evo_hip_hyena_kind kind, evo_hip_dtype dtype,
                           const void *projection, size_t length, size_t width,
                           const evo::hip::HyenaWeights &w, float *short_history,
                           float *inner_history, float *modal_state, void *workspace,
                           size_t workspace_bytes, void *output, hipStream_t s) {
  if (output == nullptr)
    return {evo::ErrorCode::kInvalidArgument, "invalid_argument: hyena output is NULL"};
  const bool planar = (static_cast<int>(dtype) & EVO_HIP_PLANAR) != 0;
  dtype = static_cast<evo_hip_dtype>(static_cast<int>(dtype) &
                                     ~(EVO_HIP_PLANAR | EVO_HIP_BF16_TAPS));
  if (dtype == EVO_HIP_F32)
    return evo::hip::hyena_forward<float, float *>(
        kind, static_cast<const float *>(projection), length, width, planar, w, short_history,
        inner_history, modal_state, workspace, workspace_bytes, static_cast<float *>(output), s);
  if (dtype == EVO_HIP_BF16)
    return evo::hip::hyena_forward<uint16_t, uint16_t *>(
        kind, static_cast<const uint16_t *>(projection), length, width, planar, w, short_history,
        inner_history, modal_state, workspace, workspace_bytes,
        static_cast<uint16_t *>(output), s);
  if (dtype == EVO_HIP_F16)
    return evo::hip::hyena_forward<float, evo::hip::F16Out>(
        kind, static_cast<const float *>(projection), length, width, planar, w, short_history,
        inner_history, modal_state, workspace, workspace_bytes,
        evo::hip::F16Out{static_cast<uint16_t *>(output)}, s);
  if (dtype == EVO_HIP_BF16_F16)
    return evo::hip::hyena_forward<uint16_t, evo::hip::F16Out>(
        kind, static_cast<const uint16_t *>(projection), length, width, planar, w, short_history,
        inner_history, modal_state, workspace, workspace_bytes,
        evo::hip::F16Out{static_cast<uint16_t *>(output)}, s);
  auto *hi = static_cast<uint16_t *>(output);
  const evo::hip::SplitOut split{hi, hi + length * width};
  if (dtype == EVO_HIP_SPLIT)
    return evo::hip::hyena_forward<float, evo::hip::SplitOut>(
        kind, static_cast<const float *>(projection), length, width, planar, w, short_history,
        inner_history, modal_state, workspace, workspace_bytes, split, s);
  if (dtype == EVO_HIP_BF16_SPLIT)
    return evo::hip::hyena_forward<uint16_t, evo::hip::SplitOut>(
        kind, static_cast<const uint16_t *>(projection), length, width, planar, w, short_history,
        inner_history, modal_state, workspace, workspace_bytes, split, s);
  return {evo::ErrorCode::kInvalidArgument, "invalid_argument: unknown dtype"};
}
}  // namespace

evo_status evo_hip_hyena_forward(evo_hip_hyena_kind kind, evo_hip_dtype dtype,
                                 const void *projection, size_t length, size_t width,
                                 const uint16_t *short_filter, size_t short_len,
                                 const float *inner_filter, size_t groups, size_t inner_len,
                                 const float *direct, const float *poles,
                                 const float *residues, size_t state_size,
                                 float *short_history, float *inner_history,
                                 float *modal_state, void *workspace, size_t workspace_bytes,
                                 void *output, void *stream) {
  return protect([&]() -> evo_status {
    const bool taps_bf16 = (static_cast<int>(dtype) & EVO_HIP_BF16_TAPS) != 0;
    const evo::hip::HyenaWeights w{short_filter, short_len, inner_filter, groups, inner_len,
                                   direct, poles, residues, state_size, taps_bf16};
    return publish(hyena_dispatch(kind, dtype, projection, length, width, w, short_history,
                                  inner_history, modal_state, workspace, workspace_bytes,
                                  output, static_cast<hipStream_t>(stream)));
  });
}

size_t evo_hip_hyena_static_scratch_bytes(void) { return evo::hip::kHyenaStaticScratchBytes; }

evo_status evo_hip_hyena_forward_static(evo_hip_hyena_kind kind, evo_hip_dtype dtype,
                                        const void *projection, size_t length, size_t width,
                                        const uint16_t *short_filter, size_t short_len,
                                        const float *inner_filter, size_t groups,
                                        size_t inner_len, const float *direct,
                                        const float *poles, const float *residues,
                                        size_t state_size, float *short_history,
                                        float *inner_history, float *modal_state, void *output,
                                        void *stream) {
  return protect([&]() -> evo_status {
    void *scratch = nullptr;
    const auto found = evo::hip::hyena_static_scratch(&scratch);
    if (!found.ok())
      return publish(found);
    const bool taps_bf16 = (static_cast<int>(dtype) & EVO_HIP_BF16_TAPS) != 0;
    const evo::hip::HyenaWeights w{short_filter, short_len, inner_filter, groups, inner_len,
                                   direct, poles, residues, state_size, taps_bf16};
    // Only the paths that keep data in a workspace (the three-pass HCL
    // fallback's chunk states, the F32-tap Toeplitz table) use the scratch;
    // each checks its need against the scratch's size before any launch.
    const evo::Status status =
        hyena_dispatch(kind, dtype, projection, length, width, w, short_history, inner_history,
                       modal_state, scratch, evo::hip::kHyenaStaticScratchBytes, output,
                       static_cast<hipStream_t>(stream));
    if (!status.ok() && status.message().find("workspace too small") != std::string::npos)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: this shape's path needs " +
                         std::to_string(evo::hip::hyena_workspace_bytes(
                             static_cast<int>(kind), length, width, state_size)) +
                         " bytes of workspace, more than the static scratch's " +
                         std::to_string(evo::hip::kHyenaStaticScratchBytes) +
                         "; use evo_hip_hyena_forward with a workspace");
    return publish(status);
  });
}

evo_status evo_hip_e4m3_quantize(evo_hip_dtype dtype, const void *x, size_t count,
                                 float scale, uint8_t *codes, void *stream) {
  return protect([&]() -> evo_status {
    const auto s = static_cast<hipStream_t>(stream);
    if (dtype == EVO_HIP_F32)
      return publish(evo::hip::e4m3_quantize_f32(static_cast<const float *>(x), count, scale,
                                                 codes, s));
    if (dtype == EVO_HIP_BF16)
      return publish(evo::hip::e4m3_quantize_bf16(static_cast<const uint16_t *>(x), count,
                                                  scale, codes, s));
    return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: unknown dtype");
  });
}

evo_status evo_hip_fp8_linear(const uint8_t *in_codes, const uint8_t *w_codes, float *out,
                              size_t m, size_t n, size_t k, float output_scale, int mode,
                              void *stream) {
  return protect([&]() -> evo_status {
    if (mode < 0 || mode > 2)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: unknown FP8 mode");
    return publish(evo::hip::fp8_linear(in_codes, w_codes, out, m, n, k, output_scale,
                                        static_cast<evo::hip::Fp8Mode>(mode),
                                        static_cast<hipStream_t>(stream)));
  });
}

evo_status evo_hip_fp8_linear_bf16(const uint8_t *in_codes, const uint8_t *w_codes,
                                   uint16_t *out, size_t m, size_t n, size_t k,
                                   float output_scale, int mode, void *stream) {
  return protect([&]() -> evo_status {
    if (mode < 0 || mode > 2)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: unknown FP8 mode");
    return publish(evo::hip::fp8_linear(in_codes, w_codes, out, m, n, k, output_scale,
                                        static_cast<evo::hip::Fp8Mode>(mode),
                                        static_cast<hipStream_t>(stream)));
  });
}

evo_status evo_hip_split_f32(const float *x, size_t count, uint16_t *hi, uint16_t *lo,
                            void *stream) {
  return protect([&]() -> evo_status {
    return publish(evo::hip::split_planes(x, count, hi, lo, static_cast<hipStream_t>(stream)));
  });
}

evo_status evo_hip_linear(const uint16_t *x_hi, const uint16_t *x_lo, const uint16_t *w,
                          const uint16_t *bias, const float *residual, size_t m, size_t n,
                          size_t k, float *out, void *stream) {
  return protect([&]() -> evo_status {
    const evo::hip::GemmEpilogue mode =
        bias != nullptr ? (residual != nullptr ? evo::hip::kGemmBiasResidual : evo::hip::kGemmBias)
                        : (residual != nullptr ? evo::hip::kGemmResidual : evo::hip::kGemmStore);
    return publish(evo::hip::gemm_bf16w(evo::hip::Activation{x_hi, x_lo, k}, w,
                                        evo::hip::GemmOutput{out, nullptr, nullptr, n}, m, n,
                                        k, mode, bias, residual, false, 0,
                                        static_cast<hipStream_t>(stream)));
  });
}

evo_status evo_hip_linear_normed(const float *x, size_t m, size_t k, const float *scale,
                                 float eps, int split, const uint16_t *w, size_t n, float *out,
                                 void *stream) {
  return protect([&]() -> evo_status {
    return publish(evo::hip::gemm_bf16w_normed(
        evo::hip::RowNorm{x, scale, eps, k}, split != 0, w,
        evo::hip::GemmOutput{out, nullptr, nullptr, n}, m, n, k, evo::hip::kGemmStore, nullptr,
        nullptr, false, 0, static_cast<hipStream_t>(stream)));
  });
}

evo_status evo_hip_fp8_linear_normed(const float *x, size_t m, size_t k, const float *scale,
                                     float eps, float input_scale, const uint8_t *w_codes,
                                     size_t n, float output_scale, int mode, uint16_t *out,
                                     void *stream) {
  return protect([&]() -> evo_status {
    if (mode != 0 && mode != 1)
      return publish({evo::ErrorCode::kInvalidArgument,
                      "invalid_argument: evo_hip_fp8_linear_normed takes modes 0 and 1"});
    return publish(evo::hip::fp8_linear_normed(
        evo::hip::RowNorm{x, scale, eps, k}, input_scale, w_codes, out, m, n, k, output_scale,
        mode == 0 ? evo::hip::kFp8MfmaK32 : evo::hip::kFp8MfmaK128,
        static_cast<hipStream_t>(stream)));
  });
}

evo_status evo_hip_linear_split(const uint16_t *x_hi, const uint16_t *x_lo, const uint16_t *w,
                                const uint16_t *bias, const float *residual, size_t m,
                                size_t n, size_t k, float *out, float *workspace,
                                size_t workspace_bytes, void *stream) {
  return protect([&]() -> evo_status {
    const evo::hip::GemmEpilogue mode =
        bias != nullptr ? (residual != nullptr ? evo::hip::kGemmBiasResidual : evo::hip::kGemmBias)
                        : (residual != nullptr ? evo::hip::kGemmResidual : evo::hip::kGemmStore);
    return publish(evo::hip::gemm_bf16w(evo::hip::Activation{x_hi, x_lo, k}, w,
                                        evo::hip::GemmOutput{out, nullptr, nullptr, n}, m, n,
                                        k, mode, bias, residual, false, 0,
                                        static_cast<hipStream_t>(stream), workspace,
                                        workspace_bytes));
  });
}

evo_status evo_hip_pack_mlp(const uint16_t *l1, const uint16_t *l2, size_t inner,
                            size_t width, uint16_t *w12, void *stream) {
  return protect([&]() -> evo_status {
    if (l1 == nullptr || l2 == nullptr || w12 == nullptr || inner == 0 || width == 0)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: invalid MLP pack");
    const size_t padded = (inner + 31) / 32 * 32;
    const auto s = static_cast<hipStream_t>(stream);
    const size_t row = width * 2;
    hipError_t e = hipMemsetAsync(w12, 0, 2 * padded * row, s);
    for (size_t q = 0; q < padded / 32 && e == hipSuccess; ++q) {
      const size_t rows = std::min<size_t>(32, inner - q * 32);
      e = hipMemcpyAsync(w12 + 64 * q * width, l1 + q * 32 * width, rows * row,
                         hipMemcpyDeviceToDevice, s);
      if (e == hipSuccess)
        e = hipMemcpyAsync(w12 + (64 * q + 32) * width, l2 + q * 32 * width, rows * row,
                           hipMemcpyDeviceToDevice, s);
    }
    if (e != hipSuccess)
      return publish(EVO_STATUS_HIP, std::string("hip: pack MLP: ") + hipGetErrorString(e));
    return publish(evo::Status::Ok());
  });
}

evo_status evo_hip_gated_mlp(const uint16_t *x_hi, const uint16_t *x_lo, const uint16_t *w12,
                             const uint16_t *l3, size_t m, size_t width, size_t inner, int gelu,
                             uint16_t *inner_workspace, const float *residual, float *out,
                             void *stream) {
  return protect([&]() -> evo_status {
    if (inner_workspace == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: MLP workspace is null");
    const size_t padded = (inner + 31) / 32 * 32;
    const auto s = static_cast<hipStream_t>(stream);
    uint16_t *inner_lo = x_lo != nullptr ? inner_workspace + m * inner : nullptr;
    auto status = evo::hip::gemm_bf16w(
        evo::hip::Activation{x_hi, x_lo, width}, w12,
        evo::hip::GemmOutput{nullptr, inner_workspace, inner_lo, inner}, m, 2 * padded, width,
        evo::hip::kGemmGated, nullptr, nullptr, gelu != 0, inner, s);
    if (!status.ok())
      return publish(status);
    return publish(evo::hip::gemm_bf16w(
        evo::hip::Activation{inner_workspace, inner_lo, inner}, l3,
        evo::hip::GemmOutput{out, nullptr, nullptr, width}, m, width, inner,
        residual != nullptr ? evo::hip::kGemmResidual : evo::hip::kGemmStore, nullptr,
        residual, false, 0, s));
  });
}

evo_status evo_hip_rms_norm(const float *x, size_t rows, size_t width, const float *scale,
                            float eps, float *out, uint16_t *out_hi, uint16_t *out_lo,
                            void *stream) {
  return protect([&]() -> evo_status {
    return publish(evo::hip::rms_norm(x, rows, width, scale, eps, out, out_hi, out_lo,
                                      static_cast<hipStream_t>(stream)));
  });
}

evo_status evo_hip_rms_norm_e4m3(const float *x, size_t rows, size_t width,
                                 const float *scale, float eps, float code_scale,
                                 uint8_t *codes, void *stream) {
  return protect([&]() -> evo_status {
    if (codes == nullptr)
      return publish(EVO_STATUS_INVALID_ARGUMENT, "invalid_argument: codes are null");
    return publish(evo::hip::rms_norm(x, rows, width, scale, eps, nullptr, nullptr, nullptr,
                                      static_cast<hipStream_t>(stream), codes, code_scale));
  });
}

evo_status evo_hip_attention(const float *projected, size_t rows, size_t width, size_t heads,
                             int column_split, const float *inv_freq, float rope_scale,
                             size_t prefix, uint16_t *query, uint16_t *key_cache,
                             uint16_t *value_cache, size_t capacity, float *out,
                             void *stream) {
  return evo_hip_attention_ws(projected, rows, width, heads, column_split, inv_freq, rope_scale,
                              prefix, query, key_cache, value_cache, capacity, out, nullptr, 0,
                              stream);
}

evo_status evo_hip_attention_ws(const float *projected, size_t rows, size_t width, size_t heads,
                                int column_split, const float *inv_freq, float rope_scale,
                                size_t prefix, uint16_t *query, uint16_t *key_cache,
                                uint16_t *value_cache, size_t capacity, float *out,
                                float *workspace, size_t workspace_bytes, void *stream) {
  return protect([&]() -> evo_status {
    const auto s = static_cast<hipStream_t>(stream);
    if (prefix + rows > capacity || capacity % 64 != 0)
      return publish(EVO_STATUS_INVALID_ARGUMENT,
                     "invalid_argument: attention rows exceed the cache capacity, or the "
                     "capacity is not a multiple of 64");
    auto status = evo::hip::qkv_rope(projected, rows, width, heads, column_split != 0,
                                     inv_freq, rope_scale, prefix, query, rows * width,
                                     key_cache, value_cache, capacity * width, capacity, s);
    if (!status.ok())
      return publish(status);
    return publish(evo::hip::causal_attention(query, rows * width, key_cache, value_cache,
                                              capacity * width, capacity, rows, prefix, heads,
                                              heads == 0 ? 0 : width / heads, out, nullptr,
                                              nullptr, s, workspace, workspace_bytes));
  });
}

}  // extern "C"
