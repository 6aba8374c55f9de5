// SPDX-License-Identifier: Apache-2.0
//
// evo-hip: command-line front end over the evo C ABI (include/evo/evo.h).
//
//   evo-hip bench -m MODEL --input FILE [--warmup N --repetitions N]
//   evo-hip score -m MODEL --input FILE [--dump-logits OUT.npy]
//   evo-hip run   -m MODEL -p DNA -n TOKENS [sampling] [--output-format raw|fasta]
//
// Subcommands, option meanings, limits and report lines follow evo.cpp's CLI:
// `bench` times a whole prefill with host logits per record and writes one
// schema-1 JSONL report (reference `src/cpu/inference_cli.cpp:400-460`,
// `src/benchmark.cpp:41-103`); `score` writes one JSON line of per-token
// log-likelihoods per record (reference `src/cpu/inference_cli.cpp:204-290,
// 358-398`); `run` prefills the prompt, decodes and samples (reference
// `src/cpu/inference_cli.cpp:292-356`).
//
// The library is opened at run time: by default libevo_hip.so beside this
// program (../lib/), or any library exporting the evo C ABI named by
// --library, so the same front end drives evo.cpp's CPU library for
// side-by-side checks. `--backend` picks the backend the library is asked for.
#include <dlfcn.h>

#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <optional>
#include <string>
#include <vector>

#include "evo/evo.h"
#include "sequence_input.hpp"

namespace evo_hip_cli {
namespace {

// ---------------------------------------------------------------- status ---

struct Status {
  int code = 0;
  std::string message;
  bool ok() const { return code == 0; }
};

constexpr int kInvalid = EVO_STATUS_INVALID_ARGUMENT;
constexpr int kIo = EVO_STATUS_IO;
constexpr int kInternal = EVO_STATUS_INTERNAL;

Status invalid(std::string message) { return {kInvalid, std::move(message)}; }

const char *code_name(int code) {
  switch (code) {
  case EVO_STATUS_INVALID_ARGUMENT:
    return "invalid_argument";
  case EVO_STATUS_IO:
    return "io";
  case EVO_STATUS_MODEL_FORMAT:
    return "model_format";
  case EVO_STATUS_UNSUPPORTED:
    return "unsupported";
  case EVO_STATUS_CUDA:
    return "cuda";
  case EVO_STATUS_MPS:
    return "mps";
  case EVO_STATUS_HIP:
    return "hip";
  default:
    return "internal";
  }
}

// ------------------------------------------------------- library binding ---

// The evo C ABI entry points this program calls, resolved from the library.
struct Api {
  void *handle = nullptr;
  const char *(*last_error)();
  const char *(*backend_name)(evo_backend);
  evo_model_params (*model_default_params)();
  evo_context_params (*context_default_params)();
  evo_sampler_params (*sampler_default_params)();
  evo_status (*model_load)(const char *, const evo_model_params *, evo_model **);
  void (*model_free)(evo_model *);
  evo_backend (*model_backend)(const evo_model *);
  const char *(*model_id)(const evo_model *);
  const char *(*model_architecture)(const evo_model *);
  const char *(*model_profile)(const evo_model *);
  size_t (*model_vocab_size)(const evo_model *);
  evo_status (*model_encode)(const evo_model *, const uint8_t *, size_t,
                             uint32_t *, size_t, size_t *);
  evo_status (*model_decode_token)(const evo_model *, uint32_t, uint8_t *);
  evo_status (*context_create)(const evo_model *, const evo_context_params *,
                               evo_context **);
  void (*context_free)(evo_context *);
  const char *(*context_profile)(const evo_context *);
  evo_status (*context_prefill)(evo_context *, const evo_batch *,
                                evo_logits_callback, void *);
  evo_status (*context_decode)(evo_context *, uint32_t, evo_logits_callback,
                               void *);
  evo_status (*batch_create)(size_t, evo_batch **);
  void (*batch_free)(evo_batch *);
  evo_status (*batch_add_sequence)(evo_batch *, const uint8_t *, size_t);
  evo_status (*sampler_create)(const evo_sampler_params *, evo_sampler **);
  void (*sampler_free)(evo_sampler *);
  evo_status (*sampler_sample)(evo_sampler *, const float *, size_t, uint32_t *);
};

template <typename F> bool bind(void *handle, const char *name, F *slot) {
  void *symbol = dlsym(handle, name);
  *slot = reinterpret_cast<F>(symbol);
  return symbol != nullptr;
}

Status open_library(const std::string &path, Api *api) {
  api->handle = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
  if (api->handle == nullptr) {
    const char *why = dlerror();
    return {kIo, "cannot load evo library '" + path + "': " +
                     (why != nullptr ? why : "unknown error")};
  }
  void *h = api->handle;
  const bool complete =
      bind(h, "evo_last_error", &api->last_error) &&
      bind(h, "evo_backend_name", &api->backend_name) &&
      bind(h, "evo_model_default_params", &api->model_default_params) &&
      bind(h, "evo_context_default_params", &api->context_default_params) &&
      bind(h, "evo_sampler_default_params", &api->sampler_default_params) &&
      bind(h, "evo_model_load", &api->model_load) &&
      bind(h, "evo_model_free", &api->model_free) &&
      bind(h, "evo_model_backend", &api->model_backend) &&
      bind(h, "evo_model_id", &api->model_id) &&
      bind(h, "evo_model_architecture", &api->model_architecture) &&
      bind(h, "evo_model_profile", &api->model_profile) &&
      bind(h, "evo_model_vocab_size", &api->model_vocab_size) &&
      bind(h, "evo_model_encode", &api->model_encode) &&
      bind(h, "evo_model_decode_token", &api->model_decode_token) &&
      bind(h, "evo_context_create", &api->context_create) &&
      bind(h, "evo_context_free", &api->context_free) &&
      bind(h, "evo_context_profile", &api->context_profile) &&
      bind(h, "evo_context_prefill", &api->context_prefill) &&
      bind(h, "evo_context_decode", &api->context_decode) &&
      bind(h, "evo_batch_create", &api->batch_create) &&
      bind(h, "evo_batch_free", &api->batch_free) &&
      bind(h, "evo_batch_add_sequence", &api->batch_add_sequence) &&
      bind(h, "evo_sampler_create", &api->sampler_create) &&
      bind(h, "evo_sampler_free", &api->sampler_free) &&
      bind(h, "evo_sampler_sample", &api->sampler_sample);
  if (!complete)
    return {kIo, "library '" + path + "' does not export the evo C ABI"};
  return {};
}

Status from_evo(const Api &api, evo_status status, const std::string &where) {
  if (status == EVO_STATUS_OK)
    return {};
  const char *message = api.last_error();
  return {static_cast<int>(status),
          where + ": " + (message != nullptr ? message : "")};
}

// --------------------------------------------------------------- options ---

enum class Command { kBench, kScore, kRun };
enum class OutputFormat { kRaw, kFasta };

struct Options {
  Command command = Command::kScore;
  std::string library;
  std::string model_path;
  std::string input_path;
  std::string prompt;
  std::string profile;
  std::optional<std::string> dump_logits;
  evo_backend backend = EVO_BACKEND_HIP;
  bool fp8_projections = false;
  size_t context_size = 8192;
  size_t warmup = 1;
  size_t repetitions = 5;
  size_t generated_tokens = 0;
  std::optional<size_t> force_prompt_threshold;
  float temperature = 1.0f;
  size_t top_k = 1;
  float top_p = 1.0f;
  uint64_t seed = 0;
  bool sampling_set = false;
  OutputFormat output_format = OutputFormat::kRaw;
  std::string generation_name = "generated";
  bool format_set = false;
};

void print_help() {
  std::fputs(
      "evo-hip - StripedHyena2 prefill/score/generation on MI355X (HIP)\n\n"
      "Usage:\n"
      "  evo-hip bench -m MODEL --input FASTA_FASTQ_OR_TEXT [--warmup N "
      "--repetitions N]\n"
      "  evo-hip score -m MODEL --input FASTA_FASTQ_OR_TEXT [--dump-logits "
      "OUT.npy]\n"
      "  evo-hip run -m MODEL -p DNA -n TOKENS [sampling] [--output-format "
      "raw|fasta --name NAME]\n\n"
      "Common options:\n"
      "  -m, --model PATH      evo2-runtime-v1 Safetensors artifact\n"
      "  --ctx N               Context size in tokens, [1, 1048576] "
      "(default: 8192)\n"
      "  --profile P           hip-f32 (default) or hip-bf16, then any of\n"
      "                        +fp8-exact | +fp8-k32, +f16-out, +f16-proj (hip-f32\n"
      "                        only), e.g. hip-f32+f16-out; exact for --backend cpu\n"
      "  --fp8-projections     Convert BF16 Hyena projections to E4M3 at load\n"
      "  --backend hip|cpu     Backend requested from the library (default: "
      "hip)\n"
      "  --library PATH        Library exporting the evo C ABI (default: "
      "libevo_hip.so)\n\n"
      "Benchmark:\n"
      "  --warmup N            Unmeasured prefill runs, [0, 1000] (default: 1)\n"
      "  --repetitions N       Measured prefill runs, [1, 10000] (default: 5)\n\n"
      "Generation:\n"
      "  -p, --prompt DNA      Prompt bytes\n"
      "  -n, --tokens N        Tokens to generate, [1, 1048576]\n"
      "  --temp T              Positive temperature (default: 1)\n"
      "  --top-k K             Keep K logits; 0 disables, 1 is greedy "
      "(default: 1)\n"
      "  --top-p P             Nucleus probability in (0,1] (default: 1)\n"
      "  --seed N              Unsigned 64-bit seed (default: 0)\n"
      "  --force-prompt-threshold N  Prompt tokens prefilled before decoding\n"
      "                        the rest one by one (default: min(3000, ctx))\n"
      "  --output-format raw|fasta, --name NAME\n"
      "  --dump-logits OUT.npy Write every step's logits (score: every "
      "row)\n",
      stdout);
}

bool parse_size(const std::string &text, uint64_t limit, uint64_t *out) {
  if (text.empty() || text.size() > 20)
    return false;
  uint64_t value = 0;
  for (const char c : text) {
    if (c < '0' || c > '9')
      return false;
    const uint64_t digit = static_cast<uint64_t>(c - '0');
    if (value > (UINT64_MAX - digit) / 10)
      return false;
    value = value * 10 + digit;
  }
  if (value > limit)
    return false;
  *out = value;
  return true;
}

bool parse_float(const std::string &text, float *out) {
  if (text.empty())
    return false;
  char *end = nullptr;
  const float value = std::strtof(text.c_str(), &end);
  if (end != text.c_str() + text.size() || !std::isfinite(value))
    return false;
  *out = value;
  return true;
}

Status parse_options(int argc, char **argv, Options *options) {
  if (argc < 2)
    return invalid("expected a command: bench, score or run");
  const std::string command = argv[1];
  if (command == "bench")
    options->command = Command::kBench;
  else if (command == "score")
    options->command = Command::kScore;
  else if (command == "run")
    options->command = Command::kRun;
  else
    return invalid("unknown command '" + command + "'");

  std::vector<std::string> seen;
  bool seen_tokens = false;
  for (int index = 2; index < argc; ++index) {
    const std::string option = argv[index];
    if (option == "--fp8-projections") {
      options->fp8_projections = true;
      continue;
    }
    if (std::find(seen.begin(), seen.end(), option) != seen.end())
      return invalid(option + " was given more than once");
    seen.push_back(option);
    if (index + 1 >= argc)
      return invalid(option + " requires a value");
    const std::string value = argv[++index];
    uint64_t number = 0;
    if (option == "-m" || option == "--model") {
      options->model_path = value;
    } else if (option == "--input") {
      options->input_path = value;
    } else if (option == "--library") {
      options->library = value;
    } else if (option == "--profile") {
      options->profile = value;
    } else if (option == "--backend") {
      if (value == "hip")
        options->backend = EVO_BACKEND_HIP;
      else if (value == "cpu")
        options->backend = EVO_BACKEND_CPU;
      else
        return invalid("--backend must be hip or cpu");
    } else if (option == "--ctx") {
      if (!parse_size(value, 1048576, &number) || number == 0)
        return invalid("--ctx must be an integer in [1, 1048576]");
      options->context_size = number;
    } else if (option == "--warmup") {
      if (!parse_size(value, 1000, &number))
        return invalid("--warmup must be an integer in [0, 1000]");
      options->warmup = number;
    } else if (option == "--repetitions") {
      if (!parse_size(value, 10000, &number) || number == 0)
        return invalid("--repetitions must be an integer in [1, 10000]");
      options->repetitions = number;
    } else if (option == "--dump-logits") {
      if (value.empty())
        return invalid("--dump-logits requires a path");
      options->dump_logits = value;
    } else if (option == "-p" || option == "--prompt") {
      options->prompt = value;
    } else if (option == "-n" || option == "--tokens") {
      if (!parse_size(value, 1048576, &number) || number == 0)
        return invalid("--tokens must be an integer in [1, 1048576]");
      options->generated_tokens = number;
      seen_tokens = true;
    } else if (option == "--temp") {
      if (!parse_float(value, &options->temperature) ||
          options->temperature <= 0.0f)
        return invalid("--temp must be a positive finite number");
      options->sampling_set = true;
    } else if (option == "--top-k") {
      if (!parse_size(value, SIZE_MAX, &number))
        return invalid("--top-k must be a nonnegative integer");
      options->top_k = number;
      options->sampling_set = true;
    } else if (option == "--top-p") {
      if (!parse_float(value, &options->top_p) || options->top_p <= 0.0f ||
          options->top_p > 1.0f)
        return invalid("--top-p must be in (0, 1]");
      options->sampling_set = true;
    } else if (option == "--seed") {
      if (!parse_size(value, UINT64_MAX, &number))
        return invalid("--seed must be an unsigned 64-bit integer");
      options->seed = number;
      options->sampling_set = true;
    } else if (option == "--force-prompt-threshold") {
      if (!parse_size(value, 1048576, &number) || number == 0)
        return invalid("--force-prompt-threshold must be a positive integer");
      options->force_prompt_threshold = number;
    } else if (option == "--output-format") {
      if (value == "raw")
        options->output_format = OutputFormat::kRaw;
      else if (value == "fasta")
        options->output_format = OutputFormat::kFasta;
      else
        return invalid("--output-format must be raw or fasta");
      options->format_set = true;
    } else if (option == "--name") {
      if (value.empty() || value.find_first_of("\r\n") != std::string::npos)
        return invalid("--name must be nonempty and single-line");
      options->generation_name = value;
      options->format_set = true;
    } else {
      return invalid("unknown option '" + option + "'");
    }
  }
  if (options->model_path.empty())
    return invalid("-m MODEL is required");
  const bool generation = options->command == Command::kRun;
  if (generation) {
    if (options->prompt.empty())
      return invalid("generation prompt must not be empty");
    if (!seen_tokens)
      return invalid("generation requires -n TOKENS");
    if (!options->input_path.empty())
      return invalid("run takes -p PROMPT, not --input");
    if (options->prompt.size() > options->context_size ||
        options->generated_tokens >
            options->context_size - options->prompt.size())
      return invalid("prompt bytes plus generated tokens exceed --ctx");
  } else {
    if (options->input_path.empty())
      return invalid(command + " requires --input FILE");
    if (!options->prompt.empty() || seen_tokens)
      return invalid("-p and -n are only valid for run");
    if (options->sampling_set || options->force_prompt_threshold)
      return invalid("sampling options are only valid for run");
    if (options->format_set)
      return invalid("--output-format and --name are only valid for run");
  }
  if (options->command == Command::kBench && options->dump_logits)
    return invalid("--dump-logits is not valid for bench");
  if (options->command != Command::kBench &&
      (std::find(seen.begin(), seen.end(), "--warmup") != seen.end() ||
       std::find(seen.begin(), seen.end(), "--repetitions") != seen.end()))
    return invalid("--warmup and --repetitions are only valid for bench");
  return {};
}

Status context_flags(const Options &options, uint32_t *flags) {
  *flags = 0;
  const std::string &p = options.profile;
  if (options.backend == EVO_BACKEND_CPU) {
    if (!p.empty() && p != "exact")
      return invalid("--backend cpu supports --profile exact only");
    return {};
  }
  if (p.empty())
    return {};
  // A base profile and '+'-separated options, as the library names the
  // context's profile (evo_context_profile).
  size_t start = 0;
  bool first = true;
  while (start <= p.size()) {
    const size_t end = std::min(p.find('+', start), p.size());
    const std::string part = p.substr(start, end - start);
    if (first && part == "hip-f32") {
    } else if (first && part == "hip-bf16") {
      *flags |= EVO_CONTEXT_FLAG_HIP_BF16;
    } else if (!first && part == "fp8-exact" && !(*flags & EVO_CONTEXT_FLAG_HIP_FP8_K32)) {
      *flags |= EVO_CONTEXT_FLAG_HIP_FP8_EXACT;
    } else if (!first && part == "fp8-k32" && !(*flags & EVO_CONTEXT_FLAG_HIP_FP8_EXACT)) {
      *flags |= EVO_CONTEXT_FLAG_HIP_FP8_K32;
    } else if (!first && part == "f16-out" && !(*flags & EVO_CONTEXT_FLAG_HIP_BF16)) {
      *flags |= EVO_CONTEXT_FLAG_HIP_F16_OUT;
    } else if (!first && part == "f16-proj" && !(*flags & EVO_CONTEXT_FLAG_HIP_BF16)) {
      *flags |= EVO_CONTEXT_FLAG_HIP_F16_PROJ;
    } else {
      *flags = 0;
      return invalid("unknown --profile '" + p + "'");
    }
    first = false;
    start = end + 1;
  }
  return {};
}

// --------------------------------------------------------------- session ---

struct Session {
  const Api *api = nullptr;
  evo_model *model = nullptr;
  size_t vocab = 0;
  ~Session() {
    if (model != nullptr)
      api->model_free(model);
  }
};

Status load_model(const Api &api, const Options &options, Session *session) {
  session->api = &api;
  evo_model_params params = api.model_default_params();
  params.backend = options.backend;
  if (options.fp8_projections)
    params.flags |= EVO_MODEL_FLAG_HIP_FP8_PROJECTIONS;
  Status status = from_evo(
      api, api.model_load(options.model_path.c_str(), &params, &session->model),
      "model load");
  if (!status.ok())
    return status;
  session->vocab = api.model_vocab_size(session->model);
  return {};
}

// One context, freed on scope exit.
struct ContextHandle {
  const Api *api;
  evo_context *context = nullptr;
  explicit ContextHandle(const Api *a) : api(a) {}
  ~ContextHandle() {
    if (context != nullptr)
      api->context_free(context);
  }
};

Status create_context(const Session &session, const Options &options,
                      ContextHandle *handle) {
  evo_context_params params = session.api->context_default_params();
  params.context_size = options.context_size;
  Status status = context_flags(options, &params.flags);
  if (!status.ok())
    return status;
  return from_evo(*session.api,
                  session.api->context_create(session.model, &params,
                                              &handle->context),
                  "context create");
}

Status encode(const Session &session, const std::string &bytes,
              std::vector<uint32_t> *tokens) {
  tokens->assign(bytes.size(), 0);
  size_t count = 0;
  Status status = from_evo(
      *session.api,
      session.api->model_encode(session.model,
                                reinterpret_cast<const uint8_t *>(bytes.data()),
                                bytes.size(), tokens->data(), tokens->size(),
                                &count),
      "encode");
  tokens->resize(count);
  return status;
}

// Whole-sequence prefill through evo_context_prefill; the library splits the
// sequence into chunks and calls `callback` once per chunk.
Status prefill(const Session &session, evo_context *context,
               const std::string &bytes, evo_logits_callback callback,
               void *user) {
  evo_batch *batch = nullptr;
  Status status =
      from_evo(*session.api, session.api->batch_create(1, &batch), "batch");
  if (!status.ok())
    return status;
  status = from_evo(
      *session.api,
      session.api->batch_add_sequence(
          batch, reinterpret_cast<const uint8_t *>(bytes.data()), bytes.size()),
      "batch");
  if (status.ok())
    status = from_evo(*session.api,
                      session.api->context_prefill(context, batch, callback, user),
                      "prefill");
  session.api->batch_free(batch);
  return status;
}

// ------------------------------------------------------------------ JSON ---

void json_string(std::string *out, const std::string &value) {
  static const char hex[] = "0123456789abcdef";
  out->push_back('"');
  for (const char raw : value) {
    const auto byte = static_cast<unsigned char>(raw);
    switch (byte) {
    case '"':
      *out += "\\\"";
      break;
    case '\\':
      *out += "\\\\";
      break;
    case '\b':
      *out += "\\b";
      break;
    case '\f':
      *out += "\\f";
      break;
    case '\n':
      *out += "\\n";
      break;
    case '\r':
      *out += "\\r";
      break;
    case '\t':
      *out += "\\t";
      break;
    default:
      if (byte < 0x20 || byte >= 0x7f) {
        *out += "\\u00";
        out->push_back(hex[byte >> 4]);
        out->push_back(hex[byte & 15]);
      } else {
        out->push_back(static_cast<char>(byte));
      }
    }
  }
  out->push_back('"');
}

// Shortest-round-trip-free 17-significant-digit form, as an ostream with
// precision 17 in default float notation prints a double.
void json_double(std::string *out, double value) {
  char text[40];
  std::snprintf(text, sizeof(text), "%.17g", value);
  *out += text;
}

Status write_stdout(const std::string &text) {
  if (std::fwrite(text.data(), 1, text.size(), stdout) != text.size() ||
      std::fflush(stdout) != 0)
    return {kIo, "failed writing to stdout"};
  return {};
}

// NPY v1.0, little-endian float32, C order [rows, columns].
Status write_npy(const std::string &path, const std::vector<float> &values,
                 size_t rows, size_t columns) {
  std::string header = "{'descr': '<f4', 'fortran_order': False, 'shape': (" +
                       std::to_string(rows) + ", " + std::to_string(columns) +
                       "), }";
  const size_t unpadded = 10 + header.size() + 1;
  header.append((64 - unpadded % 64) % 64, ' ');
  header.push_back('\n');
  std::FILE *file = std::fopen(path.c_str(), "wb");
  if (file == nullptr)
    return {kIo, "cannot open NPY output '" + path + "'"};
  const unsigned char prefix[10] = {0x93, 'N', 'U', 'M', 'P', 'Y', 1, 0,
                                    static_cast<unsigned char>(header.size() & 255),
                                    static_cast<unsigned char>(header.size() >> 8)};
  bool good = std::fwrite(prefix, 1, 10, file) == 10 &&
              std::fwrite(header.data(), 1, header.size(), file) == header.size() &&
              std::fwrite(values.data(), sizeof(float), values.size(), file) ==
                  values.size();
  good = std::fclose(file) == 0 && good;
  return good ? Status{} : Status{kIo, "failed writing NPY output '" + path + "'"};
}

// ----------------------------------------------------------------- score ---

// log softmax(logits)[target] in double: the row maximum in F32, each
// exp(F32 difference) accumulated in double
// (reference `src/cpu/inference_cli.cpp:204-222`).
bool log_probability(const float *logits, size_t columns, uint32_t target,
                     double *result) {
  float maximum = -INFINITY;
  for (size_t i = 0; i < columns; ++i) {
    if (!std::isfinite(logits[i]))
      return false;
    maximum = std::max(maximum, logits[i]);
  }
  double denominator = 0.0;
  for (size_t i = 0; i < columns; ++i)
    denominator += std::exp(static_cast<double>(logits[i] - maximum));
  *result = static_cast<double>(logits[target] - maximum) - std::log(denominator);
  return true;
}

struct ScoreState {
  const std::vector<uint32_t> *tokens;
  std::vector<double> scores;
  std::vector<float> *dump;
  size_t vocab;
  bool non_finite = false;
  bool bad_target = false;
};

evo_status score_rows(const float *logits, size_t rows, size_t columns,
                      size_t offset, void *user) {
  auto *state = static_cast<ScoreState *>(user);
  const auto &tokens = *state->tokens;
  if (columns != state->vocab)
    return EVO_STATUS_INTERNAL;
  if (state->dump != nullptr)
    state->dump->insert(state->dump->end(), logits, logits + rows * columns);
  const size_t scored =
      offset + rows < tokens.size() ? rows : tokens.size() - 1 - offset;
  const size_t base = state->scores.size();
  if (base != offset)
    return EVO_STATUS_INTERNAL;
  state->scores.resize(base + scored);
  int failures = 0;
#pragma omp parallel for schedule(static) reduction(+ : failures)
  for (long row = 0; row < static_cast<long>(scored); ++row) {
    const uint32_t target = tokens[offset + static_cast<size_t>(row) + 1];
    if (target >= columns) {
      failures += 1 << 16;
      continue;
    }
    if (!log_probability(logits + static_cast<size_t>(row) * columns, columns,
                         target, &state->scores[base + static_cast<size_t>(row)]))
      failures += 1;
  }
  if (failures != 0) {
    state->bad_target = failures >= (1 << 16);
    state->non_finite = !state->bad_target;
    return EVO_STATUS_INTERNAL;
  }
  return EVO_STATUS_OK;
}

Status run_score(const Api &api, const Options &options) {
  Session session;
  Status status = load_model(api, options, &session);
  if (!status.ok())
    return status;
  size_t records = 0;
  const InputError input = read_sequences(
      options.input_path, options.context_size,
      [&](const SequenceRecord &record) -> InputError {
        if (record.bytes.size() < 2)
          return {kInvalid,
                  "score record '" + record.name + "' must contain two bytes"};
        if (records != 0 && options.dump_logits)
          return {kInvalid, "--dump-logits requires exactly one input record"};
        ContextHandle context(&api);
        Status inner = create_context(session, options, &context);
        std::vector<uint32_t> tokens;
        if (inner.ok())
          inner = encode(session, record.bytes, &tokens);
        std::vector<float> dump;
        ScoreState state{&tokens, {}, options.dump_logits ? &dump : nullptr,
                         session.vocab};
        state.scores.reserve(tokens.size());
        if (inner.ok())
          inner = prefill(session, context.context, record.bytes, score_rows,
                          &state);
        if (!inner.ok()) {
          if (state.non_finite)
            return {kInternal, "inference backend produced non-finite logits"};
          if (state.bad_target)
            return {kInvalid, "score target exceeds vocabulary"};
          return {inner.code, inner.message};
        }
        if (state.scores.size() + 1 != tokens.size())
          return {kInternal, "inference backend returned incomplete logits"};
        if (options.dump_logits) {
          inner = write_npy(*options.dump_logits, dump, tokens.size(),
                            session.vocab);
          if (!inner.ok())
            return {inner.code, inner.message};
        }
        double total = 0.0;
        for (const double s : state.scores)
          total += s;
        const double mean = total / static_cast<double>(state.scores.size());
        std::string line = "{\"name\":";
        json_string(&line, record.name);
        line += ",\"input_format\":\"";
        line += format_name(record.format);
        line += "\",\"backend\":\"";
        line += api.backend_name(api.model_backend(session.model));
        line += "\",\"profile\":\"";
        line += api.context_profile(context.context);
        line += "\",\"model_id\":";
        json_string(&line, api.model_id(session.model));
        line += ",\"tokens\":" + std::to_string(record.bytes.size()) +
                ",\"scored_tokens\":" + std::to_string(state.scores.size()) +
                ",\"log_likelihood\":";
        json_double(&line, total);
        line += ",\"mean_log_likelihood\":";
        json_double(&line, mean);
        line += ",\"perplexity\":";
        json_double(&line, std::exp(-mean));
        line += ",\"token_log_likelihoods\":[";
        for (size_t i = 0; i < state.scores.size(); ++i) {
          if (i != 0)
            line.push_back(',');
          json_double(&line, state.scores[i]);
        }
        line += "]}\n";
        inner = write_stdout(line);
        if (!inner.ok())
          return {inner.code, inner.message};
        ++records;
        return {};
      });
  return {input.code, input.message};
}

// ----------------------------------------------------------------- bench ---

evo_status keep_nothing(const float *, size_t, size_t, size_t, void *) {
  return EVO_STATUS_OK;
}

double median(std::vector<double> values) {
  std::sort(values.begin(), values.end());
  const size_t middle = values.size() / 2;
  return values.size() % 2 == 0 ? (values[middle - 1] + values[middle]) / 2.0
                                : values[middle];
}

Status run_bench(const Api &api, const Options &options) {
  Session session;
  Status status = load_model(api, options, &session);
  if (!status.ok())
    return status;
  const InputError input = read_sequences(
      options.input_path, options.context_size,
      [&](const SequenceRecord &record) -> InputError {
        std::vector<uint32_t> tokens;
        Status inner = encode(session, record.bytes, &tokens);
        if (!inner.ok())
          return {inner.code, inner.message};
        std::string profile;
        // One measurement: a fresh context (not timed) and one whole prefill
        // with host logits (timed).
        const auto measure = [&](double *elapsed) -> Status {
          ContextHandle context(&api);
          Status s = create_context(session, options, &context);
          if (!s.ok())
            return s;
          profile = api.context_profile(context.context);
          const auto start = std::chrono::steady_clock::now();
          s = prefill(session, context.context, record.bytes, keep_nothing,
                      nullptr);
          const auto stop = std::chrono::steady_clock::now();
          if (elapsed != nullptr)
            *elapsed = std::chrono::duration<double>(stop - start).count();
          return s;
        };
        for (size_t i = 0; i < options.warmup; ++i) {
          inner = measure(nullptr);
          if (!inner.ok())
            return {inner.code,
                    "benchmark warmup " + std::to_string(i) + ": " + inner.message};
        }
        std::vector<double> samples;
        for (size_t i = 0; i < options.repetitions; ++i) {
          double elapsed = 0.0;
          inner = measure(&elapsed);
          if (!inner.ok())
            return {inner.code, "benchmark repetition " + std::to_string(i) +
                                    ": " + inner.message};
          if (!std::isfinite(elapsed) || elapsed <= 0.0)
            return {kInternal,
                    "benchmark produced a nonpositive or nonfinite duration"};
          samples.push_back(elapsed);
        }
        const double middle = median(samples);
        char identity[40];
        std::snprintf(identity, sizeof(identity), "fnv1a64:%016llx",
                      fnv1a64(record.bytes));
        std::string line = "{\"schema_version\":1,\"command\":\"bench\",\"model_path\":";
        json_string(&line, options.model_path);
        line += ",\"model_id\":";
        const char *id = api.model_id(session.model);
        if (id == nullptr || *id == '\0')
          line += "null";
        else
          json_string(&line, id);
        line += ",\"architecture\":";
        json_string(&line, api.model_architecture(session.model));
        line += ",\"artifact_profile\":";
        json_string(&line, api.model_profile(session.model));
        line += ",\"execution_profile\":";
        json_string(&line, profile);
        line += ",\"backend\":";
        json_string(&line, api.backend_name(api.model_backend(session.model)));
        line += ",\"input\":{\"path\":";
        json_string(&line, options.input_path);
        line += ",\"name\":";
        json_string(&line, record.name);
        line += ",\"format\":\"";
        line += format_name(record.format);
        line += "\",\"identity\":";
        json_string(&line, identity);
        line += "},\"context_size\":" + std::to_string(options.context_size) +
                ",\"warmup\":" + std::to_string(options.warmup) +
                ",\"repetitions\":" + std::to_string(options.repetitions) +
                ",\"tokens\":" + std::to_string(tokens.size()) +
                ",\"timing_scope\":\"prefill_with_host_logits\",\"samples_seconds\":[";
        for (size_t i = 0; i < samples.size(); ++i) {
          if (i != 0)
            line.push_back(',');
          json_double(&line, samples[i]);
        }
        line += "],\"statistic\":\"median\",\"median_seconds\":";
        json_double(&line, middle);
        line += ",\"median_tokens_per_second\":";
        json_double(&line, static_cast<double>(tokens.size()) / middle);
        line += "}\n";
        inner = write_stdout(line);
        return {inner.code, inner.message};
      });
  return {input.code, input.message};
}

// ------------------------------------------------------------------- run ---

struct LastRow {
  std::vector<float> *row;
};

evo_status keep_last_row(const float *logits, size_t rows, size_t columns,
                         size_t, void *user) {
  auto *last = static_cast<LastRow *>(user);
  if (rows == 0)
    return EVO_STATUS_INTERNAL;
  last->row->assign(logits + (rows - 1) * columns, logits + rows * columns);
  return EVO_STATUS_OK;
}

bool is_iupac_dna(char c) {
  switch (c >= 'a' && c <= 'z' ? static_cast<char>(c - 32) : c) {
  case 'A': case 'C': case 'G': case 'T': case 'R': case 'Y': case 'S':
  case 'W': case 'K': case 'M': case 'B': case 'D': case 'H': case 'V':
  case 'N':
    return true;
  default:
    return false;
  }
}

Status run_generate(const Api &api, const Options &options) {
  Session session;
  Status status = load_model(api, options, &session);
  if (!status.ok())
    return status;
  ContextHandle context(&api);
  status = create_context(session, options, &context);
  if (!status.ok())
    return status;
  std::vector<uint32_t> prompt;
  status = encode(session, options.prompt, &prompt);
  if (!status.ok())
    return status;
  // The first min(3000, ctx) prompt tokens (or --force-prompt-threshold) go
  // through prefill; the rest are decoded one by one.
  const size_t prefill_count = std::min(
      prompt.size(), options.force_prompt_threshold.value_or(
                         std::min<size_t>(3000, options.context_size)));
  std::vector<float> current;
  LastRow last{&current};
  status = prefill(session, context.context, options.prompt.substr(0, prefill_count),
                   keep_last_row, &last);
  if (!status.ok())
    return {status.code, "prompt prefill: " + status.message};
  for (size_t i = prefill_count; i < prompt.size(); ++i) {
    status = from_evo(api, api.context_decode(context.context, prompt[i],
                                              keep_last_row, &last),
                      "decode");
    if (!status.ok())
      return status;
  }
  evo_sampler_params params = api.sampler_default_params();
  params.temperature = options.temperature;
  params.top_k = options.top_k;
  params.top_p = options.top_p;
  params.seed = options.seed;
  evo_sampler *sampler = nullptr;
  status = from_evo(api, api.sampler_create(&params, &sampler), "sampler");
  if (!status.ok())
    return status;
  std::string generated;
  std::vector<float> dump;
  for (size_t step = 0; step < options.generated_tokens && status.ok(); ++step) {
    if (options.dump_logits)
      dump.insert(dump.end(), current.begin(), current.end());
    uint32_t token = 0;
    status = from_evo(api,
                      api.sampler_sample(sampler, current.data(), current.size(),
                                         &token),
                      "sample");
    uint8_t byte = 0;
    if (status.ok())
      status = from_evo(api, api.model_decode_token(session.model, token, &byte),
                        "decode token");
    if (status.ok())
      generated.push_back(static_cast<char>(byte));
    if (status.ok() && step + 1 < options.generated_tokens)
      status = from_evo(api,
                        api.context_decode(context.context, token, keep_last_row,
                                           &last),
                        "decode");
  }
  api.sampler_free(sampler);
  if (!status.ok())
    return status;
  if (options.dump_logits) {
    status = write_npy(*options.dump_logits, dump, options.generated_tokens,
                       session.vocab);
    if (!status.ok())
      return status;
  }
  if (options.output_format == OutputFormat::kRaw)
    return write_stdout(generated);
  for (size_t i = 0; i < generated.size(); ++i)
    if (!is_iupac_dna(generated[i]))
      return invalid("generated FASTA sequence contains non-IUPAC DNA byte at "
                     "offset " +
                     std::to_string(i));
  std::string text = ">" + options.generation_name + "\n";
  for (size_t offset = 0; offset < generated.size(); offset += 80)
    text += generated.substr(offset, 80) + "\n";
  return write_stdout(text);
}

std::string default_library(const char *argv0) {
  char resolved[PATH_MAX];
  std::string self = realpath("/proc/self/exe", resolved) != nullptr
                         ? std::string(resolved)
                         : std::string(argv0);
  const size_t slash = self.find_last_of('/');
  const std::string dir = slash == std::string::npos ? "." : self.substr(0, slash);
  return dir + "/../lib/libevo_hip.so";
}

} // namespace
} // namespace evo_hip_cli

int main(int argc, char **argv) {
  using namespace evo_hip_cli;
  if (argc == 2 && (std::strcmp(argv[1], "--help") == 0 ||
                    std::strcmp(argv[1], "-h") == 0)) {
    print_help();
    return 0;
  }
  Options options;
  Status status = parse_options(argc, argv, &options);
  Api api;
  if (status.ok())
    status = open_library(
        options.library.empty() ? default_library(argv[0]) : options.library,
        &api);
  if (status.ok()) {
    switch (options.command) {
    case Command::kBench:
      status = run_bench(api, options);
      break;
    case Command::kScore:
      status = run_score(api, options);
      break;
    case Command::kRun:
      status = run_generate(api, options);
      break;
    }
  }
  if (!status.ok()) {
    std::fprintf(stderr, "evo-hip: %s: %s\n", code_name(status.code),
                 status.message.c_str());
    return status.code;
  }
  return 0;
}
