// NVFP4 projections (interface of cuda/nvfp4.hpp in Enucatl/qw38) over the
// C-ABI of libqw38_hip. Elements are E2M1 nibbles, row-major [rows][pk/2]
// with element 2j in the low nibble of byte j; every 16 elements share a
// UE4M3 scale placed by the CUTLASS SM1xx swizzle over 128-row stripes. A
// weight's scales span starts with a 256-byte header whose first four bytes
// hold the FP32 global factor.
#pragma once

#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <cstdint>
#include "qw38/expected.hpp"

namespace qw38::cuda {

// Compute units of the stream's device. max_m and workspace_bytes are part
// of the interface; the HIP GEMM needs no workspace.
[[nodiscard]] expected<int, Error> prepare_nvfp4_gemm(std::uint32_t max_m, std::uint64_t workspace_bytes,
                                                      Stream const& stream);
// output FP32 [m][n] = factor * packed activation . weight rows row_start ..
// row_start + n - 1 (m <= 1024, n <= 17408, n % 8 == 0, k <= 5120,
// k % 256 == 0, row_start % 128 == 0).
[[nodiscard]] expected<void, Error> nvfp4_gemm_tile(
    void const* codes, void const* scales, std::uint8_t const* activation,
    std::uint8_t const* activation_scales, std::uint32_t m, std::uint32_t n, std::uint32_t k,
    std::uint32_t row_start, float* output, void* workspace, std::uint64_t workspace_bytes,
    int sm_count, Stream const& stream);
// BF16 [m][k] -> codes [m][pk/2] and scales of pad128(m) rows (padding rows'
// scales 0).
[[nodiscard]] expected<void, Error> launch_pack_nvfp4(std::uint16_t const* input,
                                                      std::uint8_t* codes, std::uint8_t* scales,
                                                      std::uint32_t m, std::uint32_t k,
                                                      Stream const& stream);

}  // namespace qw38::cuda
