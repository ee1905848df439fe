// One ordered HIP stream (interface of cuda/stream.hpp in Enucatl/qw38).
#pragma once

#include "cuda/device.hpp"
#include "cuda/error.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include "qw38/expected.hpp"

namespace qw38::cuda {

class Stream {
 public:
  Stream() noexcept = default;
  Stream(Stream&& other) noexcept;
  Stream& operator=(Stream&& other) noexcept;
  ~Stream();
  Stream(Stream const&) = delete;
  Stream& operator=(Stream const&) = delete;

  // A blocking stream of default priority on the current device.
  [[nodiscard]] static expected<Stream, Error> create();
  // Teardown that reports the HIP status; ownership is consumed either way.
  [[nodiscard]] expected<void, Error> close();

  [[nodiscard]] hipStream_t native() const noexcept { return stream_; }
  [[nodiscard]] bool empty() const noexcept { return stream_ == nullptr; }
  [[nodiscard]] int device() const noexcept { return device_; }

  [[nodiscard]] expected<DeviceGuard, Error> activate() const;
  [[nodiscard]] expected<void, Error> sync() const;

 private:
  Stream(hipStream_t stream, int device) noexcept : stream_(stream), device_(device) {}
  [[nodiscard]] hipError_t destroy() noexcept;
  hipStream_t stream_{nullptr};
  int device_{-1};
};

namespace testing {
// The next successful synchronisation reports a failure (after completing).
void fail_next_stream_sync() noexcept;
std::uint64_t stream_sync_count() noexcept;
}  // namespace testing

}  // namespace qw38::cuda
