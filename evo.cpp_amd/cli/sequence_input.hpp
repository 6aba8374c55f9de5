// SPDX-License-Identifier: Apache-2.0
//
// Sequence inputs of the `evo-hip` front end: raw text, FASTA and FASTQ,
// plain or gzip, path "-" for stdin. Same record rules as evo.cpp's reader
// (reference `include/evo/sequence_io.hpp:22-31`, `src/sequence_io.cpp`):
//   - first byte '>'  -> FASTA: a nonempty name per header, sequence lines
//     concatenated, blank lines ignored, no whitespace inside a line, every
//     record nonempty;
//   - first byte '@'  -> strict four-line FASTQ (@name, sequence, '+' or
//     '+name', quality of equal length in ASCII 33..126);
//   - anything else  -> one raw record named after the path ("stdin" for -).
// A record longer than `max_record_bytes` (the context size) is an error,
// found while it is read. Records are handed over one at a time.
#pragma once

#include <cstddef>
#include <functional>
#include <string>

namespace evo_hip_cli {

enum class SequenceFormat { kRaw, kFasta, kFastq };

struct SequenceRecord {
  std::string name;
  std::string bytes;
  SequenceFormat format = SequenceFormat::kRaw;
};

// Error carried out of the reader: a status code of the evo C ABI
// (2 invalid argument, 3 I/O) and a message.
struct InputError {
  int code = 0;
  std::string message;
  bool ok() const { return code == 0; }
};

using RecordCallback = std::function<InputError(const SequenceRecord &)>;

InputError read_sequences(const std::string &path, std::size_t max_record_bytes,
                          const RecordCallback &callback);

const char *format_name(SequenceFormat format);

// FNV-1a 64 of the record bytes, the benchmark input identity
// (reference `src/benchmark.cpp:30-37`).
unsigned long long fnv1a64(const std::string &bytes);

} // namespace evo_hip_cli
