// SPDX-License-Identifier: Apache-2.0
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <set>

namespace evo::hip {
namespace {

constexpr size_t kArenaRows = 8192;  // activation rows per prefill chunk
// Chunks of at most this many rows fold their RMSNorms into the few-row
// products (the gemv kernels' row limit); FP8 folding also needs W <= 8192.
constexpr size_t kFoldRows = 4;
constexpr size_t kFoldMaxWidth = 8192;
constexpr float kFp8InputAmax = 8.0F;  // activation amax of load-time FP8 conversion
// Split-K partials of short-prompt GEMMs (splits x rows x N F32; the split
// count is capped so that it fits).
constexpr size_t kSplitWorkspaceBytes = size_t{64} << 20;

Status hip_check(hipError_t error, const std::string &what) {
  if (error == hipSuccess)
    return Status::Ok();
  return {ErrorCode::kHip, "hip: " + what + ": " + hipGetErrorString(error)};
}

Status format_error(const std::string &message) {
  return {ErrorCode::kModelFormat, "model_format: " + message};
}

float bf16_host(const uint8_t *p) {
  const uint32_t bits = static_cast<uint32_t>(p[0]) << 16U | static_cast<uint32_t>(p[1]) << 24U;
  float v;
  std::memcpy(&v, &bits, 4);
  return v;
}

std::vector<float> to_f32(const TensorView &t) {
  std::vector<float> out(t.elements());
  for (size_t i = 0; i < out.size(); ++i) {
    if (t.dtype == DType::kF32)
      std::memcpy(&out[i], t.data + 4 * i, 4);
    else
      out[i] = bf16_host(t.data + 2 * i);
  }
  return out;
}

Status view(const Artifact &a, const std::string &name,
            std::vector<uint64_t> shape, DType dtype, const TensorView **out,
            bool accept_f32 = false, bool accept_fp8 = false) {
  const TensorView *t = a.tensor(name);
  if (t == nullptr)
    return format_error("required tensor is missing: " + name);
  if (t->shape != shape)
    return format_error("tensor shape mismatch: " + name);
  if (t->dtype != dtype && !(accept_f32 && t->dtype == DType::kF32) &&
      !(accept_fp8 && t->dtype == DType::kE4M3))
    return format_error("tensor dtype mismatch: " + name);
  *out = t;
  return Status::Ok();
}

Status upload_view(DeviceBuffer *buffer, const TensorView &t, const std::string &name) {
  EVO_TRY(buffer->allocate(t.bytes, name.c_str()));
  return buffer->upload(t.data, t.bytes, name.c_str());
}

Status upload_f32(DeviceBuffer *buffer, const std::vector<float> &values,
                  const std::string &name) {
  EVO_TRY(buffer->allocate(values.size() * 4, name.c_str()));
  return buffer->upload(values.data(), values.size() * 4, name.c_str());
}

}  // namespace

Status DeviceBuffer::allocate(size_t bytes, const char *what) {
  reset();
  if (bytes == 0)
    return Status::Ok();
  const hipError_t error = hipMalloc(&ptr_, bytes);
  if (error != hipSuccess) {
    ptr_ = nullptr;
    return {ErrorCode::kHip, std::string("hip: allocate ") + what + " (" +
                                 std::to_string(bytes) + " B): " + hipGetErrorString(error)};
  }
  bytes_ = bytes;
  return Status::Ok();
}

Status DeviceBuffer::upload(const void *host, size_t bytes, const char *what) {
  if (bytes > bytes_)
    return {ErrorCode::kInternal, std::string("upload overflows ") + what};
  return hip_check(hipMemcpy(ptr_, host, bytes, hipMemcpyHostToDevice),
                   std::string("upload ") + what);
}

void DeviceBuffer::reset() {
  if (ptr_ != nullptr)
    (void)hipFree(ptr_);
  ptr_ = nullptr;
  bytes_ = 0;
}

// ---------------------------------------------------------------- Model load
// Tensor set, shapes and dtypes: evo.cpp `src/cpu/model.cpp:2651-2874`.
namespace {
// FP16 copy of a BF16 weight for the one-pass FP16 products (widths that
// are a multiple of 32, the tiled kernel's K step; others keep BF16 only).
Status make_f16_copy(const DeviceBuffer &bf16, size_t count, DeviceBuffer *f16,
                     const char *what) {
  if (count % 32 != 0)
    return Status::Ok();
  EVO_TRY(f16->allocate(count * 2, what));
  EVO_TRY(bf16_to_f16(bf16.as<uint16_t>(), count, f16->as<uint16_t>(), nullptr));
  return hip_check(hipDeviceSynchronize(), what);
}
}  // namespace

Status Model::load(const Artifact &a, int device, bool allow_synthetic,
                   bool fp8_projections) {
  device_ = device;
  EVO_TRY(hip_check(hipSetDevice(device), "select device"));
  ModelConfig &c = config_;
  EVO_TRY(a.meta_string("model.architecture", &c.architecture));
  if (c.architecture == "StripedHyena2Test") {
    bool synthetic = false;
    EVO_TRY(a.meta_bool("fixture.synthetic", &synthetic));
    if (!synthetic || !allow_synthetic)
      return {ErrorCode::kUnsupported,
              "unsupported: synthetic model fixtures require explicit test permission"};
  } else if (c.architecture != "StripedHyena2") {
    return {ErrorCode::kUnsupported, "unsupported: architecture is not StripedHyena2"};
  }
  if (!a.meta_string("model.id", &c.model_id).ok())
    EVO_TRY(a.meta_string("model.name", &c.model_id));
  const std::pair<const char *, size_t *> sizes[] = {
      {"config.vocab_size", &c.vocab},
      {"config.hidden_size", &c.width},
      {"config.num_layers", &c.layers},
      {"config.num_attention_heads", &c.heads},
      {"config.state_size", &c.state},
      {"config.inner_mlp_size", &c.inner},
      {"config.short_filter_length", &c.short_len},
      {"config.hcs_filter_length", &c.hcs_len},
      {"config.hcm_filter_length", &c.hcm_len},
      {"config.hcs_filter_groups", &c.hcs_groups},
      {"config.hcm_filter_groups", &c.hcm_groups}};
  for (const auto &item : sizes) {
    uint64_t v = 0;
    EVO_TRY(a.meta_u64(item.first, &v));
    *item.second = static_cast<size_t>(v);
  }
  if (c.architecture == "StripedHyena2Test") {
    c.max_seqlen = std::numeric_limits<size_t>::max();
  } else {
    uint64_t v = 0;
    EVO_TRY(a.meta_u64("config.max_seqlen", &v));
    c.max_seqlen = static_cast<size_t>(v);
  }
  double eps = 0, rope = 0;
  EVO_TRY(a.meta_f64("config.eps", &eps));
  EVO_TRY(a.meta_f64("config.rotary_emb_scaling_factor", &rope));
  c.eps = static_cast<float>(eps);
  c.rope_scale = static_cast<float>(rope);
  if (a.has_meta("config.column_split"))
    EVO_TRY(a.meta_bool("config.column_split", &c.column_split));
  if (c.vocab == 0 || c.width == 0 || c.layers == 0 || c.heads == 0 ||
      c.width % c.heads != 0 || c.head_dim() % 2 != 0 || c.state == 0 ||
      c.state > 16 || c.inner == 0 || c.short_len < 2 || c.short_len > 8 ||
      c.hcs_len < 2 || c.hcs_len > 8 || c.hcm_len < 2 || c.hcm_len > 128 ||
      c.hcs_groups == 0 || c.hcm_groups == 0 || c.width % c.hcs_groups != 0 ||
      c.width % c.hcm_groups != 0 || !std::isfinite(c.eps) || c.eps <= 0.0F ||
      !std::isfinite(c.rope_scale) || c.rope_scale <= 0.0F || c.width % 32 != 0 ||
      c.inner % 8 != 0)
    return {ErrorCode::kUnsupported,
            "unsupported: model dimensions are outside the HIP backend's envelope "
            "(width % 32, inner % 8, state <= 16, short/HCS taps <= 8, HCM taps <= 128)"};
  const size_t hd = c.head_dim();
  if (hd != 16 && hd != 32 && hd != 64 && hd != 128)
    return {ErrorCode::kUnsupported, "unsupported: head_dim must be 16, 32, 64 or 128"};
  c.inner_padded = (c.inner + 31) / 32 * 32;

  std::vector<uint64_t> hcs, hcm, hcl, attn;
  EVO_TRY(a.meta_list("config.hcs_layer_idxs", &hcs));
  EVO_TRY(a.meta_list("config.hcm_layer_idxs", &hcm));
  EVO_TRY(a.meta_list("config.hcl_layer_idxs", &hcl));
  EVO_TRY(a.meta_list("config.attn_layer_idxs", &attn));
  layer.clear();
  layer.resize(c.layers);
  std::set<uint64_t> seen;
  auto classify = [&](const std::vector<uint64_t> &list, Mixer type,
                      const char *name) -> Status {
    for (auto index : list) {
      if (index >= c.layers || !seen.insert(index).second)
        return format_error(std::string("invalid ") + name + " layer list");
      layer[index].type = type;
    }
    return Status::Ok();
  };
  EVO_TRY(classify(hcs, Mixer::kHcs, "HCS"));
  EVO_TRY(classify(hcm, Mixer::kHcm, "HCM"));
  EVO_TRY(classify(hcl, Mixer::kHcl, "HCL"));
  EVO_TRY(classify(attn, Mixer::kAttention, "attention"));
  if (seen.size() != c.layers)
    return format_error("mixer lists do not cover all blocks");

  const size_t w = c.width;
  const TensorView *t = nullptr;
  EVO_TRY(view(a, "embedding_layer.weight", {c.vocab, w}, DType::kBF16, &t));
  EVO_TRY(upload_view(&embedding, *t, "embedding_layer.weight"));
  EVO_TRY(view(a, "norm.scale", {w}, DType::kF32, &t));
  EVO_TRY(upload_view(&final_norm, *t, "norm.scale"));

  for (size_t i = 0; i < c.layers; ++i) {
    Layer &L = layer[i];
    const std::string p = "blocks." + std::to_string(i);
    EVO_TRY(view(a, p + ".pre_norm.scale", {w}, DType::kF32, &t));
    EVO_TRY(upload_view(&L.pre_norm, *t, p + ".pre_norm.scale"));
    EVO_TRY(view(a, p + ".post_norm.scale", {w}, DType::kF32, &t));
    EVO_TRY(upload_view(&L.post_norm, *t, p + ".post_norm.scale"));
    // Gated MLP: l1 and l2 interleaved in 32-row blocks so one GEMM produces
    // both operands of every gated output in the same lane.
    const TensorView *l1 = nullptr, *l2 = nullptr, *l3 = nullptr;
    EVO_TRY(view(a, p + ".mlp.l1.weight", {c.inner, w}, DType::kBF16, &l1));
    EVO_TRY(view(a, p + ".mlp.l2.weight", {c.inner, w}, DType::kBF16, &l2));
    EVO_TRY(view(a, p + ".mlp.l3.weight", {w, c.inner}, DType::kBF16, &l3));
    {
      std::vector<uint16_t> packed(2 * c.inner_padded * w, 0);
      for (size_t q = 0; q < c.inner_padded / 32; ++q)
        for (size_t r = 0; r < 32; ++r) {
          const size_t src = q * 32 + r;
          if (src >= c.inner)
            continue;
          std::memcpy(&packed[(64 * q + r) * w], l1->data + src * w * 2, w * 2);
          std::memcpy(&packed[(64 * q + 32 + r) * w], l2->data + src * w * 2, w * 2);
        }
      EVO_TRY(L.mlp_in.allocate(packed.size() * 2, "mlp l1/l2"));
      EVO_TRY(L.mlp_in.upload(packed.data(), packed.size() * 2, "mlp l1/l2"));
    }
    EVO_TRY(upload_view(&L.mlp_out, *l3, p + ".mlp.l3.weight"));

    if (L.type == Mixer::kAttention) {
      EVO_TRY(view(a, p + ".inner_mha_cls.Wqkv.weight", {3 * w, w}, DType::kBF16, &t));
      EVO_TRY(upload_view(&L.projection, *t, p + ".Wqkv"));
      EVO_TRY(make_f16_copy(L.projection, 3 * w * w, &L.projection16, "Wqkv FP16"));
      EVO_TRY(view(a, p + ".inner_mha_cls.out_proj.weight", {w, w}, DType::kBF16, &t));
      EVO_TRY(upload_view(&L.out_weight, *t, p + ".out_proj.weight"));
      EVO_TRY(make_f16_copy(L.out_weight, w * w, &L.out_weight16, "out-projection FP16"));
      EVO_TRY(view(a, p + ".inner_mha_cls.out_proj.bias", {w}, DType::kBF16, &t));
      EVO_TRY(upload_view(&L.out_bias, *t, p + ".out_proj.bias"));
      EVO_TRY(view(a, p + ".inner_mha_cls.rotary_emb.inv_freq", {hd / 2}, DType::kF32, &t));
      EVO_TRY(upload_view(&L.inv_freq, *t, p + ".inv_freq"));
      continue;
    }
    EVO_TRY(view(a, p + ".projections.weight", {3 * w, w}, DType::kBF16, &t, false, true));
    L.fp8 = t->dtype == DType::kE4M3;
    if (!L.fp8 && fp8_projections) {
      // Load-time software-FP8 conversion of a BF16 projection, the
      // converter's per-tensor rule (`tools/evo/checkpoint.py:393-396`):
      // weight_scale = 448 / amax(W), codes = E4M3(W * weight_scale),
      // output_scale = 1 / (input_scale * weight_scale). The activation scale
      // is the fixed TE-style 448 / kFp8InputAmax.
      const auto *bits = reinterpret_cast<const uint16_t *>(t->data);
      uint16_t top = 0;
      for (uint64_t e = 0; e < t->elements(); ++e) {
        const uint16_t magnitude = bits[e] & 0x7fffU;
        if (magnitude <= 0x7f80U)  // finite or inf; NaN patterns are skipped
          top = std::max(top, magnitude);
      }
      const uint32_t wide = static_cast<uint32_t>(top) << 16U;
      float amax;
      std::memcpy(&amax, &wide, 4);
      if (!(amax > 0.0F) || !std::isfinite(amax))
        return format_error(p + ".projections.weight has no finite nonzero amax");
      const float weight_scale = 448.0F / amax;
      DeviceBuffer staging;
      EVO_TRY(upload_view(&staging, *t, p + ".projections.weight"));
      EVO_TRY(L.projection.allocate(t->elements(), "fp8 projection"));
      EVO_TRY(e4m3_quantize_bf16(staging.as<uint16_t>(), t->elements(), weight_scale,
                                 L.projection.as<uint8_t>(), nullptr));
      EVO_TRY(hip_check(hipDeviceSynchronize(), "fp8 projection conversion"));
      L.fp8 = true;
      L.fp8_input_scale = 448.0F / kFp8InputAmax;
      L.fp8_output_scale = 1.0F / (L.fp8_input_scale * weight_scale);
    } else {
      EVO_TRY(upload_view(&L.projection, *t, p + ".projections.weight"));
    }
    if (L.fp8 && t->dtype == DType::kE4M3) {
      // [input_scale, output_scale] (`src/cuda/model.cu:226-248`).
      const TensorView *s = nullptr;
      EVO_TRY(view(a, p + ".projections.fp8_runtime_scales", {2}, DType::kF32, &s));
      float scales[2];
      std::memcpy(scales, s->data, 8);
      if (!(std::isfinite(scales[0]) && scales[0] > 0 && std::isfinite(scales[1]) &&
            scales[1] > 0))
        return format_error(p + " contains invalid software-FP8 runtime scales");
      L.fp8_input_scale = scales[0];
      L.fp8_output_scale = scales[1];
    }
    if (L.fp8 && w % 32 != 0)
      return {ErrorCode::kUnsupported, "unsupported: FP8 projections need width % 32 == 0"};
    EVO_TRY(view(a, p + ".out_filter_dense.weight", {w, w}, DType::kBF16, &t));
    EVO_TRY(upload_view(&L.out_weight, *t, p + ".out_filter_dense.weight"));
    EVO_TRY(make_f16_copy(L.out_weight, w * w, &L.out_weight16, "out-projection FP16"));
    EVO_TRY(view(a, p + ".out_filter_dense.bias", {w}, DType::kBF16, &t));
    EVO_TRY(upload_view(&L.out_bias, *t, p + ".out_filter_dense.bias"));
    EVO_TRY(view(a, p + ".filter.short_filter_weight", {3 * w, 1, c.short_len}, DType::kBF16, &t));
    EVO_TRY(upload_view(&L.short_filter, *t, p + ".short_filter_weight"));
    if (L.type == Mixer::kHcs) {
      EVO_TRY(view(a, p + ".filter.h", {c.hcs_groups, 1, c.hcs_len}, DType::kBF16, &t));
      EVO_TRY(upload_f32(&L.inner_filter, to_f32(*t), p + ".filter.h"));
      continue;
    }
    EVO_TRY(view(a, p + ".filter.D", {w}, DType::kBF16, &t));
    EVO_TRY(upload_f32(&L.direct, to_f32(*t), p + ".filter.D"));
    if (L.type == Mixer::kHcm) {
      EVO_TRY(view(a, p + ".filter.h", {c.hcm_groups, 1, c.hcm_len}, DType::kBF16, &t, true));
      EVO_TRY(upload_f32(&L.inner_filter, to_f32(*t), p + ".filter.h"));
    } else {
      EVO_TRY(view(a, p + ".filter.log_poles", {w, c.state, 1}, DType::kF32, &t));
      std::vector<float> poles = to_f32(*t);
      // exp(log_pole) once, with the host libm expf the F32 reference uses
      // per step (`src/cpu/model.cpp:589-590`).
      for (auto &v : poles)
        v = std::exp(v);
      EVO_TRY(upload_f32(&L.poles, poles, p + ".poles"));
      EVO_TRY(view(a, p + ".filter.residues", {w, c.state}, DType::kF32, &t));
      EVO_TRY(upload_view(&L.residues, *t, p + ".filter.residues"));
    }
  }
  return hip_check(hipDeviceSynchronize(), "model upload");
}

// ------------------------------------------------------------------ Context
Context::~Context() {
  for (hipEvent_t event : timing_events_)
    (void)hipEventDestroy(event);
  if (host_logits_ != nullptr)
    (void)hipHostFree(host_logits_);
  if (host_flag_ != nullptr)
    (void)hipHostFree(host_flag_);
  if (stream_ != nullptr)
    (void)hipStreamDestroy(stream_);
}

Status Context::set_product_timing(bool on) {
  if (!on) {
    for (hipEvent_t event : timing_events_)
      EVO_TRY(hip_check(hipEventDestroy(event), "timing event"));
    timing_events_.clear();
    timed_pairs_ = 0;
    return Status::Ok();
  }
  if (!timing_events_.empty())
    return Status::Ok();
  timed_pairs_ = 0;
  timing_events_.resize(2 * model_->config().layers, nullptr);
  for (hipEvent_t &event : timing_events_)
    EVO_TRY(hip_check(hipEventCreate(&event), "timing event"));
  return Status::Ok();
}

Status Context::workspace_free(const char *user) const {
  if (pending_.splits != 0)
    return {ErrorCode::kInternal, std::string("internal: ") + user +
                                      " would overwrite deferred split-K partials"};
  return Status::Ok();
}

Status Context::product_time(float *ms, size_t *launches) const {
  if (ms == nullptr || launches == nullptr)
    return {ErrorCode::kInvalidArgument, "invalid_argument: null output"};
  *ms = 0.0F;
  *launches = 0;
  for (size_t i = 0; i + 1 < timing_events_.size() && i / 2 < timed_pairs_; i += 2) {
    float elapsed = 0.0F;
    EVO_TRY(hip_check(hipEventElapsedTime(&elapsed, timing_events_[i], timing_events_[i + 1]),
                      "timing event"));
    *ms += elapsed;
    ++*launches;
  }
  return Status::Ok();
}

Status Context::initialize(std::shared_ptr<const Model> model, size_t capacity,
                           const ContextOptions &options) {
  model_ = std::move(model);
  options_ = options;
  const ModelConfig &c = model_->config();
  if (capacity == 0 || capacity > c.max_seqlen)
    return {ErrorCode::kInvalidArgument,
            "invalid_argument: context requires a valid capacity"};
  capacity_ = capacity;
  cache_capacity_ = (capacity + 63) / 64 * 64;
  arena_rows_ = std::min(capacity, kArenaRows);
  // Test hook: a smaller activation arena forces multi-chunk prefill.
  // Diagnostic: GEMM classes that read only the hi plane of their split
  // activation (bit 0 BF16 projections, 1 out-projection, 2 MLP l1/l2,
  // 3 MLP l3), to measure how each class's activation rounding reaches the
  // logits. Unset (0) in every supported profile.
  if (const char *mask = std::getenv("EVO_HIP_HI_ONLY_GEMMS"))
    hi_only_ = static_cast<unsigned>(std::strtoul(mask, nullptr, 0));
  if (const char *rows = std::getenv("EVO_HIP_ARENA_ROWS")) {
    const long value = std::atol(rows);
    if (value > 0)
      arena_rows_ = std::min(arena_rows_, static_cast<size_t>(value));
  }
  profile_ = options.split_activations ? "hip-f32" : "hip-bf16";
  if (options.fp8_mode == kFp8Exact)
    profile_ += "+fp8-exact";
  else if (options.fp8_mode == kFp8MfmaK32)
    profile_ += "+fp8-k32";
  if (options.f16_proj && options.split_activations)
    profile_ += "+f16-proj";
  else if (options.f16_out && options.split_activations)
    profile_ += "+f16-out";
  EVO_TRY(hip_check(hipSetDevice(model_->device()), "select device"));
  EVO_TRY(hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "create stream"));
  const size_t R = arena_rows_, w = c.width;
  EVO_TRY(tokens_.allocate(R * 4, "tokens"));
  EVO_TRY(hidden_.allocate(R * w * 4, "hidden"));
  EVO_TRY(residual_.allocate(R * w * 4, "residual"));
  EVO_TRY(normed_.allocate(R * w * 4, "normed"));
  EVO_TRY(projected_.allocate(R * 3 * w * 4, "projection"));
  EVO_TRY(mixed_.allocate(R * w * 4, "mixer output"));
  EVO_TRY(query_.allocate(R * w * 4, "query"));
  EVO_TRY(gated_.allocate(R * c.inner * 4, "mlp gate"));
  EVO_TRY(logits_.allocate(R * c.vocab * 4, "logits"));
  EVO_TRY(codes_.allocate(R * w, "fp8 codes"));
  EVO_TRY(flag_.allocate(sizeof(int), "token and range check flag"));
  EVO_TRY(hip_check(hipMemsetAsync(flag_.as<void>(), 0, sizeof(int), stream_), "flag reset"));
  EVO_TRY(hip_check(hipHostMalloc(reinterpret_cast<void **>(&host_flag_), sizeof(int),
                                  hipHostMallocDefault), "pinned flag"));
  // Shared by the Hyena operators (chunk states, Toeplitz tables) and the
  // split-K partials of short-prompt GEMMs, which run after them.
  workspace_bytes_ = std::max({hyena_workspace_bytes(kHyenaHcl, R, w, c.state),
                               hyena_workspace_bytes(kHyenaHcs, R, w, c.state),
                               hyena_workspace_bytes(kHyenaHcm, R, w, c.state),
                               kSplitWorkspaceBytes});
  EVO_TRY(workspace_.allocate(std::max<size_t>(workspace_bytes_, 256), "hyena workspace"));
  EVO_TRY(hip_check(hipHostMalloc(reinterpret_cast<void **>(&host_logits_),
                                  R * std::max(c.vocab, w) * 4, hipHostMallocDefault),
                    "pinned logits"));
  cache_.clear();
  cache_.resize(c.layers);
  for (size_t i = 0; i < c.layers; ++i) {
    const Layer &L = model_->layer[i];
    Cache &k = cache_[i];
    if (L.type == Mixer::kAttention) {
      // split BF16 planes: K [2][capacity][W], V^T [2][W][capacity] with the
      // capacity rounded up to whole 64-key tiles; zeroed once so that tile
      // entries past the last written key are finite.
      EVO_TRY(k.keys.allocate(cache_capacity_ * w * 4, "key cache"));
      EVO_TRY(k.values.allocate(cache_capacity_ * w * 4, "value cache"));
      EVO_TRY(hip_check(hipMemsetAsync(k.keys.as<void>(), 0, k.keys.bytes(), stream_),
                        "key cache"));
      EVO_TRY(hip_check(hipMemsetAsync(k.values.as<void>(), 0, k.values.bytes(), stream_),
                        "value cache"));
      continue;
    }
    EVO_TRY(k.short_history.allocate((c.short_len - 1) * 3 * w * 4, "short FIR cache"));
    if (L.type == Mixer::kHcs)
      EVO_TRY(k.inner_history.allocate((c.hcs_len - 1) * w * 4, "HCS cache"));
    else if (L.type == Mixer::kHcm)
      EVO_TRY(k.inner_history.allocate((c.hcm_len - 1) * w * 4, "HCM cache"));
    else
      EVO_TRY(k.modal_state.allocate(w * c.state * 4, "HCL state"));
  }
  std::vector<ZeroRegion> regions;
  for (auto &k : cache_)
    for (DeviceBuffer *b : {&k.short_history, &k.inner_history, &k.modal_state})
      if (b->bytes() != 0) {
        regions.push_back(ZeroRegion{b->as<uint32_t>(), b->bytes() / 4});
        reset_max_words_ = std::max(reset_max_words_, b->bytes() / 4);
      }
  reset_count_ = regions.size();
  if (reset_count_ != 0) {
    EVO_TRY(reset_table_.allocate(reset_count_ * sizeof(ZeroRegion), "cache reset table"));
    EVO_TRY(reset_table_.upload(regions.data(), reset_count_ * sizeof(ZeroRegion),
                                "cache reset table"));
  }
  reset_caches();
  return hip_check(hipStreamSynchronize(stream_), "context initialise");
}

void Context::reset_caches() {
  // Every Hyena cache (all sizes are whole 32-bit words) in one launch.
  (void)zero_regions(reset_table_.as<ZeroRegion>(), reset_count_, reset_max_words_, stream_);
  position_ = 0;
  valid_ = false;
}

Status Context::run_layers(size_t rows, size_t capture_layer, float *capture) {
  const ModelConfig &c = model_->config();
  const size_t w = c.width;
  const bool split = options_.split_activations;
  float *hidden = hidden_.as<float>(), *residual = residual_.as<float>(),
        *projected = projected_.as<float>();
  // GEMM activations live as split BF16 planes [2][rows][cols] (lo plane
  // unused in the hip-bf16 profile).
  uint16_t *normed_hi = normed_.as<uint16_t>(), *normed_lo = normed_hi + rows * w;
  uint16_t *mixed_hi = mixed_.as<uint16_t>(), *mixed_lo = mixed_hi + rows * w;
  uint16_t *gated_hi = gated_.as<uint16_t>(), *gated_lo = gated_hi + rows * c.inner;
  const Activation normed{normed_hi, split ? normed_lo : nullptr, w};
  const Activation mixed{mixed_hi, split ? mixed_lo : nullptr, w};
  const Activation gated{gated_hi, split ? gated_lo : nullptr, c.inner};
  const SplitOut mixed_out{mixed_hi, split ? mixed_lo : nullptr};
  // Few-row chunks (decode) fold each RMSNorm into the product that reads
  // it (same values, one launch and round trip less per norm).
  const bool fold = rows <= kFoldRows;
  pending_ = SplitPartials{};
  timed_pairs_ = 0;
  for (size_t i = 0; i < c.layers; ++i) {
    const Layer &L = model_->layer[i];
    Cache &k = cache_[i];
    const RowNorm pre{hidden, L.pre_norm.as<float>(), c.eps, w};
    if (fold && pending_.splits != 0) {
      EVO_TRY(split_k_finish(pending_, hidden, rows, w, stream_));
      pending_ = SplitPartials{};
    }
    if (L.fp8) {
      const Fp8Mode mode = (w % 128 != 0) ? kFp8Exact : options_.fp8_mode;
      // The product is BF16 by definition: store it as BF16 and halve the
      // projection's HBM traffic for the Hyena kernels that read it.
      if (fold && mode != kFp8Exact && w <= kFoldMaxWidth) {
        EVO_TRY(fp8_linear_normed(pre, L.fp8_input_scale, L.projection.as<uint8_t>(),
                                  projected_.as<uint16_t>(), rows, 3 * w, w,
                                  L.fp8_output_scale, mode, stream_));
      } else {
        // The norm writes only the E4M3 codes of bf16(x) * input_scale:
        // the projection is the sole consumer of this normed activation.
        // (With pending split-K partials of the previous l3 product, the norm
        // sums them into hidden as it reads them.)
        EVO_TRY(rms_norm_partials(pending_, hidden, rows, w, L.pre_norm.as<float>(), c.eps,
                                  nullptr, nullptr, stream_, codes_.as<uint8_t>(),
                                  L.fp8_input_scale));
        pending_ = SplitPartials{};
        EVO_TRY(fp8_linear(codes_.as<uint8_t>(), L.projection.as<uint8_t>(),
                           projected_.as<uint16_t>(), rows, 3 * w, w, L.fp8_output_scale,
                           mode, stream_));
      }
    } else if (fold) {
      EVO_TRY(gemm_bf16w_normed(pre, split, L.projection.as<uint16_t>(),
                                GemmOutput{projected, nullptr, nullptr, 3 * w}, rows, 3 * w, w,
                                kGemmStore, nullptr, nullptr, false, 0, stream_));
    } else {
      EVO_TRY(rms_norm_partials(pending_, hidden, rows, w, L.pre_norm.as<float>(), c.eps,
                                normed_hi, split ? normed_lo : nullptr, stream_));
      pending_ = SplitPartials{};
      if (options_.f16_proj && split && L.projection16.bytes() != 0 && (rows * w) % 8 == 0) {
        // The normed rows as one FP16 plane (in the mixer output's buffer,
        // written only after this product) times the FP16 weight copy.
        uint16_t *normed16 = mixed_.as<uint16_t>();
        EVO_TRY(planes_to_f16(normed_hi, normed_lo, rows * w, normed16, stream_,
                              flag_.as<int>()));
        EVO_TRY(gemm_bf16w(Activation{normed16, nullptr, w, true},
                           L.projection16.as<uint16_t>(),
                           GemmOutput{projected, nullptr, nullptr, 3 * w}, rows, 3 * w, w,
                           kGemmStore, nullptr, nullptr, false, 0, stream_));
      } else {
        EVO_TRY(gemm_bf16w(hi_only_ & 1U ? Activation{normed_hi, nullptr, w} : normed,
                           L.projection.as<uint16_t>(),
                           GemmOutput{projected, nullptr, nullptr, 3 * w}, rows, 3 * w, w,
                           kGemmStore, nullptr, nullptr, false, 0, stream_));
      }
    }
    EVO_TRY(workspace_free("the mixer"));
    // "+f16-out" / "+f16-proj": the mixer writes its output as one FP16 plane
    // (fp16(v), saturating at +-65504) for the FP16 copy of the out-projection.
    const bool f16_out = (options_.f16_proj || options_.f16_out) && split && !fold &&
                         L.out_weight16.bytes() != 0;
    if (L.type == Mixer::kAttention) {
      uint16_t *query = query_.as<uint16_t>();
      const size_t cache_plane = cache_capacity_ * w;
      // With the FP16 output the range is checked on V as it enters the
      // cache (the outputs are convex combinations of V rows), not per output.
      EVO_TRY(qkv_rope(projected, rows, w, c.heads, c.column_split, L.inv_freq.as<float>(),
                       c.rope_scale, position_, query, rows * w, k.keys.as<uint16_t>(),
                       k.values.as<uint16_t>(), cache_plane, cache_capacity_, stream_,
                       f16_out ? flag_.as<int>() : nullptr));
      EVO_TRY(causal_attention(query, rows * w, k.keys.as<uint16_t>(),
                               k.values.as<uint16_t>(), cache_plane, cache_capacity_, rows,
                               position_,
                               c.heads, c.head_dim(), nullptr, mixed_out.hi, mixed_out.lo,
                               stream_, workspace_.as<float>(), workspace_.bytes(), f16_out));
    } else {
      HyenaWeights hw{};
      hw.short_filter = L.short_filter.as<uint16_t>();
      hw.short_len = c.short_len;
      hw.inner_filter = L.inner_filter.as<float>();
      hw.groups = L.type == Mixer::kHcs ? c.hcs_groups : c.hcm_groups;
      hw.inner_len = L.type == Mixer::kHcs ? c.hcs_len : c.hcm_len;
      hw.direct = L.direct.as<float>();
      hw.poles = L.poles.as<float>();
      hw.residues = L.residues.as<float>();
      hw.state = c.state;
      hw.taps_bf16 = true;  // `.filter.h` is BF16 in the artifact
      const int kind = L.type == Mixer::kHcs ? kHyenaHcs
                       : L.type == Mixer::kHcm ? kHyenaHcm : kHyenaHcl;
      auto mixer = [&](auto out) -> Status {
        using O = decltype(out);
        if (L.fp8)
          return hyena_forward<uint16_t, O>(kind, projected_.as<uint16_t>(), rows, w, false, hw,
                                            k.short_history.as<float>(),
                                            k.inner_history.as<float>(),
                                            k.modal_state.as<float>(), workspace_.as<void>(),
                                            workspace_.bytes(), out, stream_);
        return hyena_forward<float, O>(kind, projected, rows, w, false, hw,
                                       k.short_history.as<float>(), k.inner_history.as<float>(),
                                       k.modal_state.as<float>(), workspace_.as<void>(),
                                       workspace_.bytes(), out, stream_);
      };
      if (f16_out)
        EVO_TRY(mixer(F16Out{mixed_hi, flag_.as<int>()}));
      else
        EVO_TRY(mixer(mixed_out));
    }
    // residual = (mixed . Wout^T + bias) + hidden   (`src/cpu/model.cpp:641-645`)
    // Short chunks split K here; the post-mixer norm then sums the partials
    // (with bias and hidden) into residual as it reads them.
    SplitPartials out_partials;
    if (f16_out) {
      // The mixer's FP16 plane times the FP16 copy of the weight.
      EVO_TRY(gemm_bf16w(Activation{mixed_hi, nullptr, w, true}, L.out_weight16.as<uint16_t>(),
                         GemmOutput{residual, nullptr, nullptr, w}, rows, w, w,
                         kGemmBiasResidual, L.out_bias.as<uint16_t>(), hidden, false, 0,
                         stream_, workspace_.as<float>(), workspace_.bytes(), &out_partials));
    } else {
      EVO_TRY(gemm_bf16w(hi_only_ & 2U ? Activation{mixed_hi, nullptr, w} : mixed,
                         L.out_weight.as<uint16_t>(),
                         GemmOutput{residual, nullptr, nullptr, w}, rows, w, w,
                         kGemmBiasResidual, L.out_bias.as<uint16_t>(), hidden, false, 0,
                         stream_, workspace_.as<float>(), workspace_.bytes(),
                         fold ? nullptr : &out_partials));
    }
    // gated = act(l1 x) * (l2 x), act = erf-GELU in block 0 only (`:650-667`).
    // This norm stays a kernel of its own for few rows too: folded into the
    // l1/l2 product, each of its N/8 blocks (2816 at 7B) normalises the row
    // again (40 us against 6 + 32 at 7B).
    if (fold)
      EVO_TRY(rms_norm(residual, rows, w, L.post_norm.as<float>(), c.eps, nullptr, normed_hi,
                       split ? normed_lo : nullptr, stream_));
    else
      EVO_TRY(rms_norm_partials(out_partials, residual, rows, w, L.post_norm.as<float>(),
                                c.eps, normed_hi, split ? normed_lo : nullptr, stream_));
    if (!timing_events_.empty())
      EVO_TRY(hip_check(hipEventRecord(timing_events_[2 * i], stream_), "timing event"));
    EVO_TRY(gemm_bf16w(hi_only_ & 4U ? Activation{normed_hi, nullptr, w} : normed,
                       L.mlp_in.as<uint16_t>(),
                       GemmOutput{nullptr, gated_hi, split ? gated_lo : nullptr, c.inner},
                       rows, 2 * c.inner_padded, w, kGemmGated, nullptr, nullptr, i == 0,
                       c.inner, stream_, workspace_.as<float>(), workspace_.bytes()));
    if (!timing_events_.empty()) {
      EVO_TRY(hip_check(hipEventRecord(timing_events_[2 * i + 1], stream_), "timing event"));
      timed_pairs_ = i + 1;
    }
    // hidden = gated . l3^T + residual
    // Its split-K partials (short chunks) are summed by the next norm of
    // hidden, unless this layer's output is captured.
    const bool captured = capture != nullptr && capture_layer == i;
    EVO_TRY(gemm_bf16w(hi_only_ & 8U ? Activation{gated_hi, nullptr, c.inner} : gated,
                       L.mlp_out.as<uint16_t>(), GemmOutput{hidden, nullptr, nullptr, w},
                       rows, w, c.inner, kGemmResidual, nullptr, residual, false, 0, stream_,
                       workspace_.as<float>(), workspace_.bytes(),
                       fold || captured ? nullptr : &pending_));
    if (captured)
      EVO_TRY(hip_check(hipMemcpyAsync(capture, hidden, rows * w * 4,
                                       hipMemcpyDeviceToHost, stream_),
                        "capture download"));
  }
  return Status::Ok();
}

Status Context::enqueue(const uint32_t *device_tokens, size_t rows, bool initial,
                        float *device_logits, size_t capture_layer, float *capture) {
  const ModelConfig &c = model_->config();
  if (rows == 0 || rows > arena_rows_ || (device_logits == nullptr && capture == nullptr))
    return {ErrorCode::kInvalidArgument, "invalid_argument: forward arguments are invalid"};
  if (initial) {
    if (rows > capacity_)
      return {ErrorCode::kInvalidArgument, "invalid_argument: chunk exceeds capacity"};
    reset_caches();
  } else if (!valid_ || rows > capacity_ - position_) {
    return {ErrorCode::kInvalidArgument,
            "invalid_argument: continuation requires a valid prefill and free capacity"};
  }
  if (capture != nullptr && capture_layer >= c.layers)
    return {ErrorCode::kInvalidArgument, "invalid_argument: embedding layer is invalid"};
  // From here on the caches advance: the context stays invalid until the
  // caller has synchronised and confirmed success (commit()).
  valid_ = false;
  EVO_TRY(embed_tokens(device_tokens, rows, model_->embedding.as<uint16_t>(), c.vocab,
                       c.width, hidden_.as<float>(), flag_.as<int>(), stream_));
  EVO_TRY(run_layers(rows, capture_layer, capture));
  if (device_logits == nullptr || rows <= kFoldRows) {
    EVO_TRY(split_k_finish(pending_, hidden_.as<float>(), rows, c.width, stream_));
    pending_ = SplitPartials{};
  }
  if (device_logits != nullptr) {
    const GemmOutput logits{device_logits, nullptr, nullptr, c.vocab};
    if (rows <= kFoldRows) {
      EVO_TRY(gemm_bf16w_normed(
          RowNorm{hidden_.as<float>(), model_->final_norm.as<float>(), c.eps, c.width},
          options_.split_activations, model_->embedding.as<uint16_t>(), logits, rows,
          c.vocab, c.width, kGemmStore, nullptr, nullptr, false, 0, stream_));
    } else {
      uint16_t *hi = normed_.as<uint16_t>();
      uint16_t *lo = options_.split_activations ? hi + rows * c.width : nullptr;
      EVO_TRY(rms_norm_partials(pending_, hidden_.as<float>(), rows, c.width,
                                model_->final_norm.as<float>(), c.eps, hi, lo, stream_));
      pending_ = SplitPartials{};
      EVO_TRY(workspace_free("the unembedding"));
      EVO_TRY(gemm_bf16w(Activation{hi, lo, c.width}, model_->embedding.as<uint16_t>(), logits,
                         rows, c.vocab, c.width, kGemmStore, nullptr, nullptr, false, 0,
                         stream_, workspace_.as<float>(), workspace_.bytes()));
    }
  }
  position_ = initial ? rows : position_ + rows;
  return Status::Ok();
}

Status Context::finish() {
  EVO_TRY(hip_check(hipMemcpyAsync(host_flag_, flag_.as<void>(), sizeof(int),
                                   hipMemcpyDeviceToHost, stream_), "flag download"));
  EVO_TRY(hip_check(hipStreamSynchronize(stream_), "prefill"));
  if (*host_flag_ & 1)
    return {ErrorCode::kInvalidArgument, "invalid_argument: token exceeds model vocabulary"};
  if (*host_flag_ & kFlagF16Range)
    return {ErrorCode::kUnsupported,
            "unsupported: an activation of the FP16 one-pass products exceeded the FP16 "
            "range (+-65504); use a context without EVO_CONTEXT_FLAG_HIP_F16_OUT / "
            "EVO_CONTEXT_FLAG_HIP_F16_PROJ"};
  valid_ = true;
  return Status::Ok();
}

Status Context::forward(const uint32_t *tokens, size_t rows, bool initial,
                        float *logits, size_t capture_layer, float *capture) {
  const ModelConfig &c = model_->config();
  if (tokens == nullptr || rows == 0 || rows > arena_rows_)
    return {ErrorCode::kInvalidArgument, "invalid_argument: forward arguments are invalid"};
  for (size_t r = 0; r < rows; ++r)
    if (tokens[r] >= c.vocab)
      return {ErrorCode::kInvalidArgument, "invalid_argument: token exceeds model vocabulary"};
  EVO_TRY(hip_check(hipSetDevice(model_->device()), "select device"));
  EVO_TRY(hip_check(hipMemsetAsync(flag_.as<void>(), 0, sizeof(int), stream_), "flag reset"));
  EVO_TRY(hip_check(hipMemcpyAsync(tokens_.as<void>(), tokens, rows * 4,
                                   hipMemcpyHostToDevice, stream_), "token upload"));
  EVO_TRY(enqueue(tokens_.as<uint32_t>(), rows, initial,
                  logits != nullptr ? logits_.as<float>() : nullptr, capture_layer, capture));
  if (logits != nullptr)
    EVO_TRY(hip_check(hipMemcpyAsync(host_logits_, logits_.as<void>(), rows * c.vocab * 4,
                                     hipMemcpyDeviceToHost, stream_), "logits download"));
  EVO_TRY(finish());
  if (logits != nullptr && logits != host_logits_)
    std::memcpy(logits, host_logits_, rows * c.vocab * 4);
  return Status::Ok();
}

Status Context::forward_view(const uint32_t *tokens, size_t rows, bool initial,
                             const float **logits) {
  if (logits == nullptr)
    return {ErrorCode::kInvalidArgument, "invalid_argument: forward arguments are invalid"};
  // host_logits_ as the destination: the copy onto itself is skipped.
  EVO_TRY(forward(tokens, rows, initial, host_logits_, std::numeric_limits<size_t>::max(),
                  nullptr));
  *logits = host_logits_;
  return Status::Ok();
}

Status Context::prefill_resident(const uint32_t *device_tokens, size_t count,
                                 float *device_logits) {
  const ModelConfig &c = model_->config();
  if (device_tokens == nullptr || device_logits == nullptr || count == 0)
    return {ErrorCode::kInvalidArgument, "invalid_argument: resident prefill arguments"};
  if (count > capacity_)
    return {ErrorCode::kInvalidArgument,
            "invalid_argument: sequence exceeds context capacity"};
  EVO_TRY(hip_check(hipSetDevice(model_->device()), "select device"));
  EVO_TRY(hip_check(hipMemsetAsync(flag_.as<void>(), 0, sizeof(int), stream_), "flag reset"));
  for (size_t offset = 0; offset < count; offset += arena_rows_) {
    const size_t rows = std::min(arena_rows_, count - offset);
    EVO_TRY(enqueue(device_tokens + offset, rows, offset == 0,
                    device_logits + offset * c.vocab, std::numeric_limits<size_t>::max(),
                    nullptr));
    if (offset + rows < count)
      valid_ = true;  // later chunks of this call continue from it
  }
  return finish();
}

}  // namespace evo::hip
