// The hidden-state RMS producers of the projection path (the launch_hidden_rms
// and launch_hidden_rms_q8 entries of cuda/activation.hpp in Enucatl/qw38).
// The rest of that header (attention, GDN, RoPE, FP8/NVFP4 producers) is not
// part of this build.
#pragma once

#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <cstdint>
#include "qw38/expected.hpp"

namespace qw38::cuda {

// RMS over hidden 5120 -> BF16 -> Q8 pack; *failure = 1 on a nonfinite group.
[[nodiscard]] expected<void, Error> launch_hidden_rms_q8(
    float const* residual, std::uint16_t const* gamma, float eps, unsigned m,
    std::int8_t* codes, float* scales, std::int32_t* sums, int* failure, Stream const& stream);

// RMS over hidden 5120 -> BF16 [n_tokens][5120].
[[nodiscard]] expected<void, Error> launch_hidden_rms(float const* residual,
                                                           std::uint16_t const* gamma, float eps,
                                                           std::uint32_t n_tokens,
                                                           std::uint16_t* out_bf16,
                                                           Stream const& stream);

}  // namespace qw38::cuda
