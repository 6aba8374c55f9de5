// SPDX-License-Identifier: Apache-2.0
// Sequence-file reader of the evo-hip front end (record rules follow
// reference `src/sequence_io.cpp:42-300`; the code is this project's own).
#include "sequence_input.hpp"

#include <zlib.h>

#include <cstdio>
#include <cstring>
#include <limits>
#include <memory>
#include <string_view>
#include <vector>

namespace evo_hip_cli {
namespace {

constexpr int kInvalid = 2; // EVO_STATUS_INVALID_ARGUMENT
constexpr int kIo = 3;      // EVO_STATUS_IO
constexpr std::size_t kMaxHeaderBytes = std::size_t{1} << 20;

InputError invalid(std::string message) { return {kInvalid, std::move(message)}; }

// Buffered byte source over zlib's gz reader, which passes plain files
// through unchanged and inflates gzip members.
class Source {
public:
  explicit Source(gzFile file) : file_(file), buffer_(1 << 16) {}
  ~Source() {
    if (file_ != nullptr)
      gzclose(file_);
  }
  Source(const Source &) = delete;
  Source &operator=(const Source &) = delete;

  // Next byte without consuming it; -1 at end of input, -2 on a read error.
  int peek() {
    if (position_ == filled_ && !refill())
      return failed_ ? -2 : -1;
    return static_cast<unsigned char>(buffer_[position_]);
  }

  // Reads one line without its '\n'. `limit` bounds the bytes kept; a longer
  // line is an error. `has_line` is false only at end of input.
  InputError line(std::size_t limit, std::string *out, bool *has_line) {
    out->clear();
    *has_line = false;
    bool any = false;
    while (true) {
      if (position_ == filled_ && !refill()) {
        if (failed_)
          return {kIo, "failed while reading sequence input"};
        *has_line = any;
        return {};
      }
      any = true;
      const char *begin = buffer_.data() + position_;
      const char *end = buffer_.data() + filled_;
      const char *newline = static_cast<const char *>(
          memchr(begin, '\n', static_cast<std::size_t>(end - begin)));
      const std::size_t take =
          static_cast<std::size_t>((newline != nullptr ? newline : end) - begin);
      if (take > limit - out->size())
        return invalid("line exceeds the record limit");
      out->append(begin, take);
      position_ += take;
      if (newline != nullptr) {
        ++position_;
        *has_line = true;
        return {};
      }
    }
  }

  // Appends everything that is left, up to `limit` bytes in total.
  InputError rest(std::size_t limit, std::string *out, bool *too_long) {
    *too_long = false;
    while (true) {
      if (position_ == filled_ && !refill())
        return failed_ ? InputError{kIo, "failed while reading sequence input"}
                       : InputError{};
      const std::size_t take = filled_ - position_;
      if (take > limit - out->size()) {
        *too_long = true;
        return {};
      }
      out->append(buffer_.data() + position_, take);
      position_ = filled_;
    }
  }

private:
  bool refill() {
    if (failed_)
      return false;
    const int count =
        gzread(file_, buffer_.data(), static_cast<unsigned>(buffer_.size()));
    if (count < 0) {
      failed_ = true;
      return false;
    }
    position_ = 0;
    filled_ = static_cast<std::size_t>(count);
    return count > 0;
  }

  gzFile file_;
  std::vector<char> buffer_;
  std::size_t position_ = 0;
  std::size_t filled_ = 0;
  bool failed_ = false;
};

std::size_t with_cr(std::size_t limit) {
  return limit == std::numeric_limits<std::size_t>::max() ? limit : limit + 1;
}

void strip_cr(std::string *line) {
  if (!line->empty() && line->back() == '\r')
    line->pop_back();
}

bool has_inner_space(std::string_view line) {
  for (const char c : line)
    if (c == ' ' || c == '\t' || c == '\v' || c == '\f' || c == '\r')
      return true;
  return false;
}

std::string at_line(std::size_t number) { return " at line " + std::to_string(number); }

InputError read_fasta(Source &in, std::size_t max_bytes,
                      const RecordCallback &callback) {
  SequenceRecord record;
  bool open = false;
  std::size_t number = 0;
  std::string line;
  while (true) {
    const bool header = in.peek() == '>';
    const std::size_t room = open ? max_bytes - record.bytes.size() : max_bytes;
    bool has_line = false;
    InputError error = in.line(header ? kMaxHeaderBytes : with_cr(room), &line,
                               &has_line);
    if (!error.ok()) {
      if (error.code == kInvalid && !header && open)
        return invalid("FASTA record '" + record.name + "' exceeds maximum " +
                       std::to_string(max_bytes) + " bytes");
      return {error.code, error.message + at_line(number + 1)};
    }
    if (!has_line)
      break;
    ++number;
    strip_cr(&line);
    if (line.empty())
      continue;
    if (line.front() == '>') {
      if (line.size() == 1)
        return invalid("FASTA line " + std::to_string(number) +
                       " has an empty header");
      if (open && record.bytes.empty())
        return invalid("FASTA record '" + record.name + "' has no sequence");
      if (open) {
        error = callback(record);
        if (!error.ok())
          return error;
      }
      record = {line.substr(1), {}, SequenceFormat::kFasta};
      open = true;
      continue;
    }
    if (!open)
      return invalid("FASTA sequence appears before the first header" +
                     at_line(number));
    if (has_inner_space(line))
      return invalid("FASTA sequence contains whitespace" + at_line(number));
    if (line.size() > max_bytes - record.bytes.size())
      return invalid("FASTA record '" + record.name + "' exceeds maximum " +
                     std::to_string(max_bytes) + " bytes");
    record.bytes += line;
  }
  if (!open)
    return invalid("FASTA contains no records");
  if (record.bytes.empty())
    return invalid("FASTA record '" + record.name + "' has no sequence");
  return callback(record);
}

InputError read_fastq(Source &in, std::size_t max_bytes,
                      const RecordCallback &callback) {
  std::size_t number = 0;
  std::size_t records = 0;
  std::string header, sequence, plus, quality;
  while (in.peek() >= 0) {
    bool has_line = false;
    InputError error = in.line(kMaxHeaderBytes, &header, &has_line);
    ++number;
    if (!error.ok())
      return {error.code, error.message + at_line(number)};
    strip_cr(&header);
    if (!has_line || header.size() < 2 || header.front() != '@')
      return invalid("FASTQ line " + std::to_string(number) +
                     " must contain a nonempty @ header");
    const std::string name = header.substr(1);

    const auto next = [&](std::size_t limit, std::string *out,
                          const char *what) -> InputError {
      bool present = false;
      InputError inner = in.line(limit, out, &present);
      ++number;
      if (!inner.ok())
        return {inner.code, inner.message + at_line(number)};
      if (!present)
        return invalid("FASTQ record '" + name + "' is truncated before its " +
                       what);
      strip_cr(out);
      return {};
    };
    error = next(with_cr(max_bytes), &sequence, "sequence");
    if (!error.ok())
      return error.message.find("record limit") != std::string::npos
                 ? invalid("FASTQ record '" + name + "' exceeds maximum " +
                           std::to_string(max_bytes) + " bytes")
                 : error;
    if (sequence.size() > max_bytes)
      return invalid("FASTQ record '" + name + "' exceeds maximum " +
                     std::to_string(max_bytes) + " bytes");
    if (sequence.empty())
      return invalid("FASTQ sequence is empty" + at_line(number));
    if (has_inner_space(sequence))
      return invalid("FASTQ sequence contains whitespace" + at_line(number));
    error = next(kMaxHeaderBytes, &plus, "+ line");
    if (!error.ok())
      return error;
    if (plus.empty() || plus.front() != '+' ||
        (plus.size() > 1 && plus.compare(1, std::string::npos, name) != 0))
      return invalid("FASTQ + line does not match record '" + name + "'" +
                     at_line(number));
    error = next(with_cr(max_bytes), &quality, "quality");
    if (!error.ok())
      return error;
    if (quality.size() != sequence.size())
      return invalid("FASTQ record '" + name +
                     "' quality length does not match sequence" +
                     at_line(number));
    for (const char c : quality) {
      const auto value = static_cast<unsigned char>(c);
      if (value < 33 || value > 126)
        return invalid("FASTQ record '" + name +
                       "' has a quality byte outside ASCII 33..126" +
                       at_line(number));
    }
    error = callback({name, sequence, SequenceFormat::kFastq});
    if (!error.ok())
      return error;
    ++records;
  }
  if (in.peek() == -2)
    return {kIo, "failed while reading sequence input"};
  return records == 0 ? invalid("FASTQ contains no records") : InputError{};
}

InputError read_raw(Source &in, const std::string &path, std::size_t max_bytes,
                    const RecordCallback &callback) {
  SequenceRecord record{path == "-" ? "stdin" : path, {}, SequenceFormat::kRaw};
  bool too_long = false;
  InputError error = in.rest(max_bytes, &record.bytes, &too_long);
  if (!error.ok())
    return {error.code, error.message + " '" + path + "'"};
  if (too_long)
    return invalid("raw sequence '" + record.name + "' exceeds maximum " +
                   std::to_string(max_bytes) + " bytes");
  if (record.bytes.empty())
    return invalid("sequence input is empty: '" + path + "'");
  return callback(record);
}

} // namespace

InputError read_sequences(const std::string &path, std::size_t max_record_bytes,
                          const RecordCallback &callback) {
  if (path.empty())
    return invalid("sequence input path must not be empty");
  if (max_record_bytes == 0)
    return invalid("sequence record limit must be positive");
  gzFile file = path == "-" ? gzdopen(fileno(stdin), "rb")
                            : gzopen(path.c_str(), "rb");
  if (file == nullptr)
    return {kIo, "cannot open sequence input '" + path + "'"};
  Source in(file);
  const int first = in.peek();
  if (first == -2)
    return {kIo, "failed while reading sequence input '" + path + "'"};
  if (first == -1)
    return invalid("sequence input is empty: '" + path + "'");
  if (first == '>')
    return read_fasta(in, max_record_bytes, callback);
  if (first == '@')
    return read_fastq(in, max_record_bytes, callback);
  return read_raw(in, path, max_record_bytes, callback);
}

const char *format_name(SequenceFormat format) {
  switch (format) {
  case SequenceFormat::kRaw:
    return "raw";
  case SequenceFormat::kFasta:
    return "fasta";
  case SequenceFormat::kFastq:
    return "fastq";
  }
  return "unknown";
}

unsigned long long fnv1a64(const std::string &bytes) {
  unsigned long long hash = 0xcbf29ce484222325ULL;
  for (const char c : bytes) {
    hash ^= static_cast<unsigned char>(c);
    hash *= 0x100000001b3ULL;
  }
  return hash;
}

} // namespace evo_hip_cli
