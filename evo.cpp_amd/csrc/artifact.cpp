// SPDX-License-Identifier: Apache-2.0
#include "artifact.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <set>

namespace evo {
namespace {

constexpr uint64_t kMaxHeader = 16ULL << 20;

Status format_error(const std::string &message) {
  return {ErrorCode::kModelFormat, "model_format: " + message};
}

// Minimal strict JSON reader for the Safetensors header: objects, strings
// (standard escapes), unsigned integer arrays. Duplicate keys are rejected.
class HeaderReader {
public:
  HeaderReader(const char *begin, const char *end) : p_(begin), end_(end) {}

  Status parse(std::map<std::string, std::string> *metadata,
               std::map<std::string, TensorView> *tensors,
               std::vector<std::pair<uint64_t, uint64_t>> *ranges) {
    ws();
    if (!take('{'))
      return format_error("header is not a JSON object");
    std::set<std::string> keys;
    bool has_metadata = false;
    ws();
    if (take('}'))
      return format_error("header object is empty");
    while (true) {
      std::string key;
      ws();
      if (!string(&key) || !colon())
        return format_error("invalid header entry");
      if (!keys.insert(key).second)
        return format_error("duplicate header key '" + key + "'");
      if (key == "__metadata__") {
        has_metadata = true;
        ws();
        if (!take('{'))
          return format_error("__metadata__ is not an object");
        ws();
        if (!take('}')) {
          while (true) {
            std::string mkey, mvalue;
            ws();
            if (!string(&mkey) || !colon() || !string(&mvalue))
              return format_error("invalid __metadata__ entry");
            if (metadata->count(mkey))
              return format_error("duplicate metadata key '" + mkey + "'");
            (*metadata)[mkey] = mvalue;
            ws();
            if (take(','))
              continue;
            if (take('}'))
              break;
            return format_error("invalid __metadata__ object");
          }
        }
      } else {
        TensorView view;
        view.name = key;
        uint64_t begin = 0, end = 0;
        EVO_TRY(tensor(&view, &begin, &end));
        ranges->emplace_back(begin, end);
        (*tensors)[key] = view;
        view.bytes = end - begin;
        (*tensors)[key].bytes = end - begin;
        (*tensors)[key].data = reinterpret_cast<const uint8_t *>(begin);  // offset; fixed up later
      }
      ws();
      if (take(','))
        continue;
      if (take('}'))
        break;
      return format_error("expected ',' or '}' in header");
    }
    ws();
    if (p_ != end_)
      return format_error("header has trailing bytes");
    if (!has_metadata)
      return format_error("missing __metadata__");
    return Status::Ok();
  }

private:
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t'))
      ++p_;
  }
  bool take(char c) {
    if (p_ < end_ && *p_ == c) {
      ++p_;
      return true;
    }
    return false;
  }
  bool colon() {
    ws();
    const bool ok = take(':');
    ws();
    return ok;
  }
  bool string(std::string *out) {
    if (!take('"'))
      return false;
    out->clear();
    while (p_ < end_) {
      const char c = *p_++;
      if (c == '"')
        return true;
      if (static_cast<unsigned char>(c) < 0x20)
        return false;
      if (c != '\\') {
        out->push_back(c);
        continue;
      }
      if (p_ >= end_)
        return false;
      const char e = *p_++;
      switch (e) {
      case '"': case '\\': case '/': out->push_back(e); break;
      case 'n': out->push_back('\n'); break;
      case 't': out->push_back('\t'); break;
      case 'r': out->push_back('\r'); break;
      case 'b': out->push_back('\b'); break;
      case 'f': out->push_back('\f'); break;
      default: return false;
      }
    }
    return false;
  }
  bool u64(uint64_t *out) {
    ws();
    const char *start = p_;
    uint64_t value = 0;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
      const uint64_t digit = static_cast<uint64_t>(*p_ - '0');
      if (value > (UINT64_MAX - digit) / 10)
        return false;
      value = value * 10 + digit;
      ++p_;
    }
    if (p_ == start || (p_ - start > 1 && *start == '0'))
      return false;
    *out = value;
    ws();
    return true;
  }
  bool u64_array(std::vector<uint64_t> *out) {
    ws();
    if (!take('['))
      return false;
    out->clear();
    ws();
    if (take(']'))
      return true;
    while (true) {
      uint64_t value;
      if (!u64(&value))
        return false;
      out->push_back(value);
      if (take(']'))
        return true;
      if (!take(','))
        return false;
    }
  }
  Status tensor(TensorView *view, uint64_t *begin, uint64_t *end) {
    ws();
    if (!take('{'))
      return format_error("tensor descriptor is not an object");
    bool has_dtype = false, has_shape = false, has_offsets = false;
    while (true) {
      std::string field;
      ws();
      if (!string(&field) || !colon())
        return format_error("invalid tensor descriptor for '" + view->name + "'");
      if (field == "dtype" && !has_dtype) {
        std::string dtype;
        if (!string(&dtype))
          return format_error("invalid dtype for '" + view->name + "'");
        if (dtype == "F32") view->dtype = DType::kF32;
        else if (dtype == "BF16") view->dtype = DType::kBF16;
        else if (dtype == "F8_E4M3") view->dtype = DType::kE4M3;
        else return format_error("unsupported dtype '" + dtype + "' for '" + view->name + "'");
        has_dtype = true;
      } else if (field == "shape" && !has_shape) {
        if (!u64_array(&view->shape))
          return format_error("invalid shape for '" + view->name + "'");
        has_shape = true;
      } else if (field == "data_offsets" && !has_offsets) {
        std::vector<uint64_t> offsets;
        if (!u64_array(&offsets) || offsets.size() != 2)
          return format_error("invalid data_offsets for '" + view->name + "'");
        *begin = offsets[0];
        *end = offsets[1];
        has_offsets = true;
      } else {
        return format_error("unexpected tensor field '" + field + "'");
      }
      ws();
      if (take(','))
        continue;
      if (take('}'))
        break;
      return format_error("invalid tensor descriptor for '" + view->name + "'");
    }
    if (!has_dtype || !has_shape || !has_offsets)
      return format_error("incomplete tensor descriptor for '" + view->name + "'");
    if (view->shape.size() > 8 || *end <= *begin)
      return format_error("invalid rank or range for '" + view->name + "'");
    uint64_t elements = 1;
    for (auto d : view->shape) {
      if (d == 0 || elements > UINT64_MAX / d)
        return format_error("invalid dimensions for '" + view->name + "'");
      elements *= d;
    }
    const uint64_t width = view->dtype == DType::kF32 ? 4 : view->dtype == DType::kBF16 ? 2 : 1;
    if (elements > UINT64_MAX / width || elements * width != *end - *begin)
      return format_error("dtype/shape size mismatch for '" + view->name + "'");
    return Status::Ok();
  }

  const char *p_;
  const char *end_;
};

uint64_t parse_u64_text(const std::string &text, bool *ok) {
  *ok = !text.empty() && !(text.size() > 1 && text[0] == '0');
  uint64_t value = 0;
  for (char c : text) {
    if (c < '0' || c > '9' || value > (UINT64_MAX - static_cast<uint64_t>(c - '0')) / 10) {
      *ok = false;
      return 0;
    }
    value = value * 10 + static_cast<uint64_t>(c - '0');
  }
  return value;
}

}  // namespace

Artifact::~Artifact() {
  if (map_ != nullptr)
    munmap(map_, map_size_);
}

Status Artifact::open(const std::string &path) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0)
    return {ErrorCode::kIo, "io: cannot open '" + path + "': " + std::strerror(errno)};
  struct stat info {};
  if (fstat(fd, &info) != 0 || !S_ISREG(info.st_mode)) {
    ::close(fd);
    return {ErrorCode::kIo, "io: '" + path + "' is not a regular file"};
  }
  map_size_ = static_cast<size_t>(info.st_size);
  if (map_size_ < 16) {
    ::close(fd);
    return format_error("file is too short");
  }
  map_ = mmap(nullptr, map_size_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map_ == MAP_FAILED) {
    map_ = nullptr;
    return {ErrorCode::kIo, "io: mmap failed for '" + path + "'"};
  }
  const auto *bytes = static_cast<const uint8_t *>(map_);
  uint64_t header = 0;
  for (int i = 0; i < 8; ++i)
    header |= static_cast<uint64_t>(bytes[i]) << (8 * i);
  if (header == 0 || header % 8 != 0 || header > kMaxHeader || header + 8 > map_size_)
    return format_error("header size must be a nonzero 8-byte multiple at most 16 MiB inside the file");
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  HeaderReader reader(reinterpret_cast<const char *>(bytes + 8),
                      reinterpret_cast<const char *>(bytes + 8 + header));
  EVO_TRY(reader.parse(&metadata_, &tensors_, &ranges));
  if (tensors_.empty())
    return format_error("artifact holds no tensors");
  for (const auto &[key, value] : metadata_) {
    if (value.size() < 2 || value[1] != ':' ||
        std::string("sufblx").find(value[0]) == std::string::npos)
      return format_error("metadata '" + key + "' has an unknown type prefix");
  }
  const uint64_t data_offset = 8 + header;
  const uint64_t data_size = map_size_ - data_offset;
  std::sort(ranges.begin(), ranges.end());
  uint64_t cursor = 0;
  for (const auto &[begin, end] : ranges) {
    if (begin != cursor)
      return format_error("tensor data buffer contains a hole or overlap");
    cursor = end;
  }
  if (cursor != data_size)
    return format_error("tensor data does not cover the complete file");
  for (auto &[name, view] : tensors_)
    view.data = bytes + data_offset + reinterpret_cast<uint64_t>(view.data);
  std::string profile;
  if (meta_string("evo2.profile", &profile).ok())
    profile_ = profile;
  else
    return format_error("missing evo2.profile metadata");
  return Status::Ok();
}

const TensorView *Artifact::tensor(const std::string &name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

Status Artifact::meta_string(const std::string &key, std::string *out) const {
  auto it = metadata_.find(key);
  if (it == metadata_.end() || it->second.rfind("s:", 0) != 0)
    return format_error("required string metadata is missing: " + key);
  *out = it->second.substr(2);
  return Status::Ok();
}

Status Artifact::meta_u64(const std::string &key, uint64_t *out) const {
  auto it = metadata_.find(key);
  bool ok = false;
  if (it != metadata_.end() && it->second.rfind("u:", 0) == 0)
    *out = parse_u64_text(it->second.substr(2), &ok);
  if (!ok)
    return format_error("required u64 metadata is missing or invalid: " + key);
  return Status::Ok();
}

Status Artifact::meta_f64(const std::string &key, double *out) const {
  auto it = metadata_.find(key);
  if (it == metadata_.end() || it->second.size() != 18 || it->second.rfind("f:", 0) != 0)
    return format_error("required f64 metadata is missing or invalid: " + key);
  uint64_t bits = 0;
  for (size_t i = 2; i < 18; ++i) {
    const char c = it->second[i];
    uint64_t digit;
    if (c >= '0' && c <= '9') digit = static_cast<uint64_t>(c - '0');
    else if (c >= 'a' && c <= 'f') digit = static_cast<uint64_t>(c - 'a' + 10);
    else return format_error("metadata '" + key + "' has invalid f64 bits");
    bits = (bits << 4) | digit;
  }
  std::memcpy(out, &bits, sizeof(*out));
  return Status::Ok();
}

Status Artifact::meta_bool(const std::string &key, bool *out) const {
  auto it = metadata_.find(key);
  if (it == metadata_.end() || (it->second != "b:0" && it->second != "b:1"))
    return format_error("required bool metadata is missing or invalid: " + key);
  *out = it->second == "b:1";
  return Status::Ok();
}

Status Artifact::meta_list(const std::string &key, std::vector<uint64_t> *out) const {
  auto it = metadata_.find(key);
  if (it == metadata_.end() || it->second.rfind("l:", 0) != 0)
    return format_error("required list metadata is missing: " + key);
  out->clear();
  const std::string body = it->second.substr(2);
  if (body.empty())
    return Status::Ok();
  size_t start = 0;
  while (start <= body.size()) {
    size_t comma = body.find(',', start);
    if (comma == std::string::npos)
      comma = body.size();
    bool ok = false;
    out->push_back(parse_u64_text(body.substr(start, comma - start), &ok));
    if (!ok)
      return format_error("metadata '" + key + "' has an invalid u64 list");
    start = comma + 1;
  }
  return Status::Ok();
}

}  // namespace evo
