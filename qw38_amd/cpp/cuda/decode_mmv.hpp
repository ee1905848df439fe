// BF16-activation decode GEMV (interface of cuda/decode_mmv.hpp in
// Enucatl/qw38). The descriptor types, wire IDs, padding and byte-count
// helpers are the reference's; this build implements the Q4_K (0x020D), Q4G64,
// Q8G32, BF16 dense-tile, FP8 (0x020F) and NVFP4 (0x020E) layouts.
#pragma once

#include "cuda/error.hpp"
#include "cuda/stream.hpp"

#include <cstddef>
#include <cstdint>
#include "qw38/expected.hpp"
#include <limits>
#include <span>

namespace qw38::cuda {

inline constexpr int kDecodeWarps = 8;
inline constexpr int kDecodeThreads = 256;
inline constexpr int kDecodeTileRows = 8;
inline constexpr int kDecodeTileK = 256;
inline constexpr int kDecodeMaxK = 17408;
inline constexpr std::uint32_t kDecodeMaxN =
    std::numeric_limits<std::uint32_t>::max() - (static_cast<std::uint32_t>(kDecodeTileRows) - 1u);

inline constexpr std::uint16_t kDecodeLayoutQ4G64V0 = 0x0201;
inline constexpr std::uint16_t kDecodeLayoutQ8G32V0 = 0x0202;
inline constexpr std::uint16_t kDecodeLayoutBf16DenseTileV0 = 0x0203;
inline constexpr std::uint16_t kDecodeLayoutQ4G64CandidateV1 = 0x020B;
inline constexpr std::uint16_t kDecodeLayoutQ8G32CandidateV1 = 0x020C;
inline constexpr std::uint16_t kDecodeLayoutQ4KCandidateV2 = 0x020D;
inline constexpr std::uint16_t kDecodeLayoutFp8V1 = 0x020F;
inline constexpr std::uint16_t kDecodeQuantizerFp8V1 = 0x0107;
inline constexpr std::uint16_t kDecodeLayoutNvFp4V1 = 0x020E;
inline constexpr std::uint16_t kDecodeQuantizerNvFp4V1 = 0x0106;
inline constexpr std::uint16_t kDecodeQuantizerNone = 0x0100;
inline constexpr std::uint16_t kDecodeQuantizerQ4G64V0 = 0x0101;
inline constexpr std::uint16_t kDecodeQuantizerQ8G32V0 = 0x0102;
inline constexpr std::uint16_t kDecodeQuantizerQ4G64CandidateV1 = 0x0103;
inline constexpr std::uint16_t kDecodeQuantizerQ8G32CandidateV1 = 0x0104;
inline constexpr std::uint16_t kDecodeQuantizerQ4KCandidateV2 = 0x0105;

enum class DecodeActivationPolicy : std::uint8_t { Bf16 = 1 };

enum class DecodeEpilogue : std::uint8_t {
  StoreBf16 = 1,
  StoreFp32 = 2,
  ResidualAddFp32 = 3,
  // Paired gate/up only: y = BF16(SiLU(gate) * up).
  SwigluStoreBf16 = 4,
};

enum class DecodeMemorySpace : std::uint8_t {
  Device = 1,
  Host = 2,
};

enum class DecodeDtype : std::uint8_t {
  Q4 = 1,
  Q8 = 2,
  Bf16 = 3,
  Fp16 = 4,
  Fp32 = 5,
  NvFp4 = 6,
  Fp8 = 7,
};

inline constexpr std::uint16_t kDecodeLayoutBf16VectorV0 = 0x0205;
inline constexpr std::uint16_t kDecodeLayoutFp32VectorV0 = 0x020A;

// Borrowed operand metadata at the launch boundary. Matrices are [N, K];
// vectors use logical/padded N with K = 1.
struct DecodeOperandView {
  void* pointer{};
  DecodeMemorySpace space{DecodeMemorySpace::Device};
  DecodeDtype dtype{};
  std::uint16_t layout{};
  std::uint32_t logical_n{};
  std::uint32_t logical_k{};
  std::uint32_t padded_n{};
  std::uint32_t padded_k{};
  std::uint64_t bytes{};
  std::uint32_t alignment{};
  bool writable{};

  friend bool operator==(DecodeOperandView const&, DecodeOperandView const&) = default;
};

[[nodiscard]] constexpr DecodeOperandView decode_matrix_view(
    void* pointer, DecodeDtype dtype, std::uint16_t layout, std::uint32_t logical_n,
    std::uint32_t logical_k, std::uint32_t padded_n, std::uint32_t padded_k, std::uint64_t bytes,
    std::uint32_t alignment, bool writable = false,
    DecodeMemorySpace space = DecodeMemorySpace::Device) noexcept {
  return {pointer, space, dtype, layout, logical_n, logical_k, padded_n, padded_k,
          bytes, alignment, writable};
}

[[nodiscard]] constexpr DecodeOperandView decode_vector_view(
    void* pointer, DecodeDtype dtype, std::uint16_t layout, std::uint32_t elements,
    std::uint64_t bytes, std::uint32_t alignment, bool writable,
    DecodeMemorySpace space = DecodeMemorySpace::Device) noexcept {
  return {pointer, space, dtype, layout, elements, 1, elements, 1, bytes, alignment, writable};
}

// Accumulation-order budget against a sequential CPU GEMV.
namespace decode_mmv_tol {
inline constexpr float kFp32Abs = 1.0e-3f;
inline constexpr float kFp32Rel = 1.0e-4f;
inline constexpr float kBf16StoreAbs = 8.0e-3f;
}  // namespace decode_mmv_tol

struct DecodeMmvDesc {
  std::uint16_t layout{};
  std::uint16_t quantizer{};
  DecodeActivationPolicy activation_policy{DecodeActivationPolicy::Bf16};
  std::uint32_t n{};
  std::uint32_t k{};
  std::uint32_t padded_n{};
  std::uint32_t padded_k{};
  DecodeOperandView codes{};
  // Q4_K: the FP16-backed span of 16-byte super-block metadata.
  DecodeOperandView scales{};
  DecodeOperandView input{};
  DecodeOperandView output{};
  // ResidualAddFp32 reads residual and writes output when output is supplied;
  // an empty output updates the residual in place.
  DecodeOperandView residual{};
  DecodeEpilogue epilogue{DecodeEpilogue::StoreBf16};
};

struct DecodeMmvPairedDesc {
  DecodeMmvDesc a;
  DecodeMmvDesc b;
};

// Two or three projections sharing K, input and layout, BF16 stores.
struct DecodeMmvRangeDesc {
  std::span<DecodeMmvDesc const> ranges{};
};

[[nodiscard]] constexpr std::uint64_t decode_pad_n(std::uint32_t n) noexcept {
  if (n == 0) return 0;
  std::uint64_t const rem = std::uint64_t(n) % kDecodeTileRows;
  return rem == 0 ? n : std::uint64_t(n) + (kDecodeTileRows - rem);
}

[[nodiscard]] constexpr std::uint32_t decode_pad_k(std::uint32_t k) noexcept {
  if (k == 0) return 0;
  auto const rem = k % static_cast<std::uint32_t>(kDecodeTileK);
  return rem == 0 ? k : k + (static_cast<std::uint32_t>(kDecodeTileK) - rem);
}

[[nodiscard]] constexpr std::uint64_t decode_code_bytes(std::uint16_t layout,
                                                        std::uint32_t padded_n,
                                                        std::uint32_t padded_k) noexcept {
  std::uint64_t const nk = std::uint64_t(padded_n) * padded_k;
  if (layout == kDecodeLayoutNvFp4V1 || layout == kDecodeLayoutQ4G64V0 ||
      layout == kDecodeLayoutQ4G64CandidateV1 || layout == kDecodeLayoutQ4KCandidateV2)
    return nk / 2u;
  if (layout == kDecodeLayoutFp8V1) return nk;
  if (layout == kDecodeLayoutQ8G32V0 || layout == kDecodeLayoutQ8G32CandidateV1) return nk;
  if (layout == kDecodeLayoutBf16DenseTileV0) return nk * 2u;
  return 0;
}

[[nodiscard]] constexpr std::uint64_t decode_scale_bytes(std::uint16_t layout,
                                                         std::uint32_t padded_n,
                                                         std::uint32_t padded_k) noexcept {
  std::uint64_t const rows = padded_n;
  if (layout == kDecodeLayoutNvFp4V1) return 256 + ((rows + 127) / 128) * 128 * (padded_k / 16u);
  if (layout == kDecodeLayoutQ4KCandidateV2) return rows * (std::uint64_t(padded_k) / 256u) * 16u;
  if (layout == kDecodeLayoutQ4G64V0 || layout == kDecodeLayoutQ4G64CandidateV1)
    return rows * (std::uint64_t(padded_k) / 64u) * 2u;
  if (layout == kDecodeLayoutFp8V1) return (rows / 128) * (padded_k / 128) * 4;
  if (layout == kDecodeLayoutQ8G32V0 || layout == kDecodeLayoutQ8G32CandidateV1)
    return rows * (std::uint64_t(padded_k) / 32u) * 2u;
  return 0;
}

[[nodiscard]] expected<void, Error> launch_decode_mmv(DecodeMmvDesc const& desc,
                                                           Stream const& stream);
[[nodiscard]] expected<void, Error> launch_decode_mmv_paired(DecodeMmvPairedDesc const& desc,
                                                                  Stream const& stream);
// Grouped GDN a/b: two BF16 dense-tile matrices, FP32 outputs, one launch.
[[nodiscard]] expected<void, Error> launch_decode_ab_bf16(DecodeMmvPairedDesc const& desc,
                                                               Stream const& stream);
[[nodiscard]] expected<void, Error> launch_decode_mmv_ranges(DecodeMmvRangeDesc const& desc,
                                                                  Stream const& stream);

}  // namespace qw38::cuda
