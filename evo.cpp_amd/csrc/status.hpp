// SPDX-License-Identifier: Apache-2.0
// Status type of the library. Codes equal the evo_status values of
// include/evo/evo.h (reference error model: evo.cpp include/evo/status.hpp).
#pragma once

#include <string>
#include <utility>

namespace evo {

enum class ErrorCode : int {
  kOk = 0,
  kInvalidArgument = 2,
  kIo = 3,
  kModelFormat = 4,
  kUnsupported = 5,
  kCuda = 6,
  kMps = 7,
  kHip = 8,
  kInternal = 70
};

inline const char *error_code_name(const ErrorCode code) {
  switch (code) {
  case ErrorCode::kOk: return "ok";
  case ErrorCode::kInvalidArgument: return "invalid_argument";
  case ErrorCode::kIo: return "io";
  case ErrorCode::kModelFormat: return "model_format";
  case ErrorCode::kUnsupported: return "unsupported";
  case ErrorCode::kCuda: return "cuda";
  case ErrorCode::kMps: return "mps";
  case ErrorCode::kHip: return "hip";
  case ErrorCode::kInternal: return "internal";
  }
  return "unknown";
}

class Status {
public:
  Status() = default;
  Status(ErrorCode code, std::string message)
      : code_(code), message_(std::move(message)) {}
  static Status Ok() { return {}; }
  bool ok() const { return code_ == ErrorCode::kOk; }
  ErrorCode code() const { return code_; }
  const std::string &message() const { return message_; }

private:
  ErrorCode code_{ErrorCode::kOk};
  std::string message_;
};

#define EVO_TRY(expr)                                                          \
  do {                                                                         \
    ::evo::Status evo_try_status_ = (expr);                                    \
    if (!evo_try_status_.ok())                                                 \
      return evo_try_status_;                                                  \
  } while (0)

}  // namespace evo
