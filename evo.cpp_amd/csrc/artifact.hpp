// SPDX-License-Identifier: Apache-2.0
// Read-only view of a single-file evo2-runtime-v1 Safetensors artifact.
//
// Layout and validation rules follow evo.cpp's reader
// (`src/model_format.cpp:749-1223`, `docs/model-format.md`): 8-byte LE header
// length (nonzero, multiple of 8, <= 16 MiB), a JSON object with a
// `__metadata__` map of typed strings (s:/u:/f:/b:/l:/x:) and one descriptor
// per tensor (dtype F32 | BF16 | F8_E4M3, rank <= 8, positive dims), payload
// ranges that tile the data buffer exactly (no hole, overlap or trailing
// bytes).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "status.hpp"

namespace evo {

enum class DType { kF32, kBF16, kE4M3 };

struct TensorView {
  std::string name;
  DType dtype{DType::kF32};
  std::vector<uint64_t> shape;
  const uint8_t *data{nullptr};
  uint64_t bytes{0};
  uint64_t elements() const {
    uint64_t n = 1;
    for (auto d : shape)
      n *= d;
    return n;
  }
};

class Artifact {
public:
  Artifact() = default;
  ~Artifact();
  Artifact(const Artifact &) = delete;
  Artifact &operator=(const Artifact &) = delete;

  Status open(const std::string &path);

  const TensorView *tensor(const std::string &name) const;
  // Typed metadata accessors; they fail when the key is absent or its type
  // prefix differs.
  Status meta_string(const std::string &key, std::string *out) const;
  Status meta_u64(const std::string &key, uint64_t *out) const;
  Status meta_f64(const std::string &key, double *out) const;
  Status meta_bool(const std::string &key, bool *out) const;
  Status meta_list(const std::string &key, std::vector<uint64_t> *out) const;
  bool has_meta(const std::string &key) const { return metadata_.count(key) != 0; }
  const std::string &profile() const { return profile_; }

private:
  void *map_{nullptr};
  size_t map_size_{0};
  std::map<std::string, std::string> metadata_;
  std::map<std::string, TensorView> tensors_;
  std::string profile_;
};

}  // namespace evo
