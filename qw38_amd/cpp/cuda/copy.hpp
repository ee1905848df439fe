// Stream-ordered copies (interface of cuda/copy.hpp in Enucatl/qw38).
#pragma once

#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <cstddef>
#include <cstdint>
#include "qw38/expected.hpp"
#include <span>

namespace qw38::cuda {

[[nodiscard]] expected<void, Error> copy_h2d(void* dst, void const* src, std::uint64_t bytes,
                                                  Stream const& stream);
[[nodiscard]] expected<void, Error> copy_d2h(void* dst, void const* src, std::uint64_t bytes,
                                                  Stream const& stream);
[[nodiscard]] expected<void, Error> copy_d2d(void* dst, void const* src, std::uint64_t bytes,
                                                  Stream const& stream);
[[nodiscard]] expected<void, Error> copy_h2d(void* dst, std::span<std::byte const> src,
                                                  Stream const& stream);
[[nodiscard]] expected<void, Error> copy_d2h(std::span<std::byte> dst, void const* src,
                                                  Stream const& stream);
// dst[i] = seed + i (uint8 wrap), written by a fill kernel.
[[nodiscard]] expected<void, Error> fill_pattern(void* dst, std::uint64_t bytes,
                                                      std::uint8_t seed, Stream const& stream);

}  // namespace qw38::cuda
