// Status type of the domain runtime interface (same names and codes as the
// reference's include/hcp_ringattn/core/status.h:9-45, so callers written against
// that interface compile unchanged).
#pragma once

#include <sstream>
#include <string>
#include <utility>

namespace hcp_ringattn {

class Status {
 public:
  enum class Code { kOk = 0, kInvalidArgument = 1, kUnimplemented = 2, kInternal = 3 };

  Status() = default;
  static Status Ok() { return Status(); }

  template <typename... Args>
  static Status Error(Code code, Args&&... args) {
    std::ostringstream text;
    (text << ... << std::forward<Args>(args));
    return Status(code, text.str());
  }

  bool ok() const { return code_ == Code::kOk; }
  Code code() const { return code_; }
  const std::string& message() const { return message_; }

 private:
  Status(Code code, std::string message) : code_(code), message_(std::move(message)) {}
  Code code_ = Code::kOk;
  std::string message_;
};

}  // namespace hcp_ringattn
