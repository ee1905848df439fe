// The hidden-state RMS producers of the projection path (the
// launch_hidden_rms, launch_hidden_rms_q8, launch_hidden_rms_fp8 and
// launch_hidden_rms_nvfp4 entries of cuda/activation.hpp in Enucatl/qw38).
// The rest of that header (attention, GDN, RoPE) is not part of this build.
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

// RMS over hidden 5120 -> FP8: codes [pad128(n_tokens)][5120], scales
// [40][pad128(n_tokens)]; companion, when non-null, receives the BF16 rows.
[[nodiscard]] expected<void, Error> launch_hidden_rms_fp8(
    float const* residual, std::uint16_t const* gamma, float eps, std::uint32_t n_tokens,
    std::uint16_t* companion, std::uint8_t* codes, float* scales, Stream const& stream);

// RMS over hidden 5120 -> NVFP4: codes [n_tokens][2560], scales of
// pad128(n_tokens) rows.
[[nodiscard]] expected<void, Error> launch_hidden_rms_nvfp4(
    float const* residual, std::uint16_t const* gamma, float eps, std::uint32_t n_tokens,
    std::uint8_t* codes, std::uint8_t* scales, Stream const& stream);

}  // namespace qw38::cuda
