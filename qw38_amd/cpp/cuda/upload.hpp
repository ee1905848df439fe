// Host bytes -> a new device buffer (interface of cuda/upload.hpp in
// Enucatl/qw38), plus this build's typed load-time repack of GGML-order
// Q4_K / Q6_K super-blocks into the tiled layouts.
#pragma once

#include "cuda/buffer.hpp"
#include "cuda/copy.hpp"
#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <cstdint>
#include "qw38/expected.hpp"
#include <span>

namespace qw38::cuda {
struct PrefillWeight;

// Allocate a device buffer and copy host bytes onto `stream`; empty payloads
// are rejected.
[[nodiscard]] expected<DeviceBuffer, Error> upload(std::span<std::byte const> host,
                                                        Stream const& stream);

// Device-resident tiled weight produced by a typed upload: owns its codes and
// metadata and describes them as a PrefillWeight.
struct TiledWeight {
  DeviceBuffer codes;
  DeviceBuffer scales;
  std::uint16_t layout{};
  std::uint16_t quantizer{};
  std::uint32_t n{}, k{};
  [[nodiscard]] PrefillWeight weight() const;
};

// n * (k / 256) GGML-order super-blocks (144 B Q4_K, 210 B Q6_K), row-major,
// repacked on the device into `layout` (0x020D or 0x0240 for Q4_K; 0x0241
// for Q6_K). Lossless: only the byte order changes.
[[nodiscard]] expected<TiledWeight, Error> upload_q4k_blocks(
    std::span<std::byte const> blocks, std::uint32_t n, std::uint32_t k, std::uint16_t layout,
    Stream const& stream);
[[nodiscard]] expected<TiledWeight, Error> upload_q6k_blocks(
    std::span<std::byte const> blocks, std::uint32_t n, std::uint32_t k, Stream const& stream);

}  // namespace qw38::cuda
