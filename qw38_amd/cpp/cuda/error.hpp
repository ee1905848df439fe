// qw38::cuda error model (interface of cuda/error.hpp in Enucatl/qw38) on HIP.
// Error::cuda_status keeps its name and holds the hipError_t value.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include "qw38/expected.hpp"
#include <source_location>
#include <string>
#include <string_view>

namespace qw38::cuda {

enum class ErrorCode : std::uint16_t {
  Status = 1,
  InvalidArgument = 2,
  Overflow = 3,
};

struct Error {
  ErrorCode code{ErrorCode::Status};
  int cuda_status{static_cast<int>(hipSuccess)};
  std::string operation;
  std::string detail;

  friend bool operator==(Error const&, Error const&) = default;
};

[[nodiscard]] char const* code_name(ErrorCode code) noexcept;

[[nodiscard]] Error from_status(hipError_t status, std::string_view operation,
                                std::source_location loc = std::source_location::current());

[[nodiscard]] Error make_error(ErrorCode code, std::string_view operation,
                               std::string_view detail);

[[nodiscard]] std::string error_message(Error const& error);

[[nodiscard]] inline expected<void, Error> check(
    hipError_t status, std::string_view operation,
    std::source_location loc = std::source_location::current()) {
  if (status == hipSuccess) return {};
  // The status is also the sticky last error: consume it so later launches
  // do not observe a stale failure.
  (void)hipGetLastError();
  return unexpected(from_status(status, operation, loc));
}

// The C-ABI status of a libqw38_hip call as an expected, with the details of
// that call's failure (qw38_last_error) on error.
[[nodiscard]] expected<void, Error> from_abi(int status);

}  // namespace qw38::cuda
