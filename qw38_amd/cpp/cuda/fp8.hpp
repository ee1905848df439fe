// FP8 (OCP E4M3FN) projections (interface of cuda/fp8.hpp in Enucatl/qw38)
// over the C-ABI of libqw38_hip. Operands are borrowed device spans; padded
// extents are multiples of 128. A packed operand is owned by the caller until
// every consumer has completed; consumers never pack it again.
#pragma once

#include "cuda/decode_mmv.hpp"
#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <cstddef>
#include <cstdint>
#include "qw38/expected.hpp"
#include <span>

namespace qw38::cuda {

// codes [m][k] E4M3, scales [k/128][m] FP32 (one per 128-wide block of a row)
struct Fp8Input {
  std::span<std::uint8_t const> codes;
  std::span<float const> scales;
  unsigned m{}, k{};
};
// codes [n][k] E4M3, scales [k/128][n/128] FP32 (one per 128 x 128 block)
struct Fp8Weight {
  std::span<std::uint8_t const> codes;
  std::span<float const> scales;
  unsigned n{}, k{};
};

// decode_mmv of one FP8 descriptor (layout 0x020F); the descriptor is
// validated by the library exactly as launch_decode_mmv validates it.
[[nodiscard]] expected<void, Error> fp8_decode(DecodeMmvDesc const& desc, Stream const& stream);
// Compute units of the stream's device (the GEMM's persistent-grid width).
[[nodiscard]] expected<int, Error> prepare_fp8_gemm(Stream const& stream);
// FP32 -> BF16 bits, round to nearest even.
[[nodiscard]] expected<void, Error> fp8_store_bf16(std::span<float const> input,
                                                   std::span<std::uint16_t> output,
                                                   Stream const& stream);
// BF16 [m][k] -> codes [pm][pk], scales [pk/128][pm] with
// scale = max(absmax / 448, 2^-126) per 128-wide block (1 for a zero block,
// NaN for a block holding a nonfinite value).
[[nodiscard]] expected<void, Error> pack_fp8(std::span<std::uint16_t const> input, unsigned m,
                                             unsigned k, std::span<std::uint8_t> codes,
                                             std::span<float> scales, Stream const& stream);
// output [m][n] FP32 = sum over 128-blocks of (weight scale * input scale) *
// (block of codes . block of codes). workspace and sm_count are part of the
// interface; the HIP kernel uses no workspace.
[[nodiscard]] expected<void, Error> fp8_gemm(Fp8Weight weight, Fp8Input input,
                                             std::span<float> output,
                                             std::span<std::byte> workspace, int sm_count,
                                             Stream const& stream);
// output [n] FP32 = weight . BF16 input [k].
[[nodiscard]] expected<void, Error> fp8_gemv(Fp8Weight weight, std::span<std::uint16_t const> input,
                                             std::span<float> output, Stream const& stream);

}  // namespace qw38::cuda
