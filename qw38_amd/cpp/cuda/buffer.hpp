// Owned device and pinned host memory (interface of cuda/buffer.hpp in
// Enucatl/qw38).
#pragma once

#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include "qw38/expected.hpp"
#include <span>
#include <utility>

namespace qw38::cuda {

class HostBuffer {
 public:
  HostBuffer() = default;
  HostBuffer(HostBuffer&& other) noexcept : ptr_(std::exchange(other.ptr_, nullptr)) {}
  HostBuffer& operator=(HostBuffer&& other) noexcept {
    if (this != &other) {
      if (ptr_) (void)hipHostFree(ptr_);
      ptr_ = std::exchange(other.ptr_, nullptr);
    }
    return *this;
  }
  ~HostBuffer() {
    if (ptr_) (void)hipHostFree(ptr_);
  }
  HostBuffer(HostBuffer const&) = delete;
  HostBuffer& operator=(HostBuffer const&) = delete;
  static expected<HostBuffer, Error> allocate(std::size_t bytes) {
    HostBuffer result;
    if (auto st = check(hipHostMalloc(&result.ptr_, bytes, hipHostMallocDefault), "hipHostMalloc");
        !st)
      return unexpected(st.error());
    return result;
  }
  void* data() noexcept { return ptr_; }

 private:
  void* ptr_{};
};

class DeviceBuffer {
 public:
  DeviceBuffer() noexcept = default;
  DeviceBuffer(DeviceBuffer&& other) noexcept;
  DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;
  ~DeviceBuffer();
  DeviceBuffer(DeviceBuffer const&) = delete;
  DeviceBuffer& operator=(DeviceBuffer const&) = delete;

  [[nodiscard]] static expected<DeviceBuffer, Error> allocate(std::uint64_t bytes);
  [[nodiscard]] static expected<DeviceBuffer, Error> allocate(std::uint64_t bytes, int device);

  // Teardown that reports the HIP status; ownership is consumed either way.
  [[nodiscard]] expected<void, Error> close();

  [[nodiscard]] void* data() noexcept { return ptr_; }
  [[nodiscard]] void const* data() const noexcept { return ptr_; }
  [[nodiscard]] std::uint64_t bytes() const noexcept { return bytes_; }
  [[nodiscard]] bool empty() const noexcept { return ptr_ == nullptr; }
  [[nodiscard]] int device() const noexcept { return device_; }
  [[nodiscard]] std::byte* as_bytes() noexcept { return static_cast<std::byte*>(ptr_); }
  [[nodiscard]] std::byte const* as_bytes() const noexcept {
    return static_cast<std::byte const*>(ptr_);
  }

 private:
  DeviceBuffer(void* ptr, std::uint64_t bytes, int device) noexcept
      : ptr_(ptr), bytes_(bytes), device_(device) {}
  [[nodiscard]] hipError_t destroy() noexcept;
  void* ptr_{nullptr};
  std::uint64_t bytes_{0};
  int device_{-1};
};

[[nodiscard]] expected<void, Error> zero(DeviceBuffer& buffer, Stream const& stream);
[[nodiscard]] expected<void, Error> zero(void* ptr, std::uint64_t bytes, Stream const& stream);

}  // namespace qw38::cuda
