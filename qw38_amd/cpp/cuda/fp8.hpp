// FP8 operand types (interface of cuda/fp8.hpp in Enucatl/qw38). Only the
// types are part of this build: PrefillProjection carries an Fp8Input; the
// FP8 kernels are not implemented and their entry points report so.
#pragma once

#include "cuda/decode_mmv.hpp"
#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <cstdint>
#include "qw38/expected.hpp"
#include <span>

namespace qw38::cuda {

struct Fp8Input {
  std::span<std::uint8_t const> codes;
  std::span<float const> scales;
  unsigned m{}, k{};
};
struct Fp8Weight {
  std::span<std::uint8_t const> codes;
  std::span<float const> scales;
  unsigned n{}, k{};
};

[[nodiscard]] expected<void, Error> pack_fp8(std::span<std::uint16_t const> input, unsigned m,
                                                  unsigned k, std::span<std::uint8_t> codes,
                                                  std::span<float> scales, Stream const& stream);
[[nodiscard]] expected<void, Error> fp8_gemv(Fp8Weight weight,
                                                  std::span<std::uint16_t const> input,
                                                  std::span<float> output, Stream const& stream);

}  // namespace qw38::cuda
