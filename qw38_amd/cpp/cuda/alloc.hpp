// Device allocation instrumentation (interface of cuda/alloc.hpp in
// Enucatl/qw38), backed by the counters of libqw38_hip.
#pragma once

#include <cstdint>

namespace qw38::cuda {

[[nodiscard]] std::uint64_t malloc_count() noexcept;
[[nodiscard]] std::uint64_t free_count() noexcept;
[[nodiscard]] std::uint64_t live_bytes() noexcept;
[[nodiscard]] std::uint64_t peak_live_bytes() noexcept;

// Accounting for allocations made outside DeviceBuffer.
void record_malloc(std::uint64_t bytes) noexcept;
void record_free(std::uint64_t bytes) noexcept;

}  // namespace qw38::cuda
