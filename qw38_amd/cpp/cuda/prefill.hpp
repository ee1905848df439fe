// BF16 prefill engine (interface of cuda/prefill.hpp in Enucatl/qw38). Q4_K
// 0x020D weights run on this build's BF16 MFMA projection; the Q8 MMQ path is
// q4k_q8_project. Other weight layouts are rejected as not implemented.
#pragma once

#include "cuda/buffer.hpp"
#include "cuda/decode_mmv.hpp"
#include "cuda/error.hpp"
#include "cuda/fp8.hpp"
#include "cuda/stream.hpp"

#include <cstdint>
#include "qw38/expected.hpp"
#include <span>

namespace qw38::cuda {

inline constexpr std::uint32_t kPrefillMaxTokens = 1024;
inline constexpr std::uint32_t kPrefillDefaultTokens = 1024;
inline constexpr std::uint32_t kPrefillDefaultWeightRows = 512;
inline constexpr std::uint32_t kPrefillMaxK = 17408;
inline constexpr std::uint32_t kPrefillHeadRows = 8;

// Validate an externally borrowed device span before a multi-stage layer
// mutates state: device memory of `device`, aligned, inside one allocation.
[[nodiscard]] expected<void, Error> validate_prefill_device_span(void const* pointer,
                                                                      std::uint64_t bytes,
                                                                      std::uint32_t alignment,
                                                                      int device);

struct PrefillWeight {
  void const* codes{};
  void const* scales{};
  std::uint16_t layout{};
  std::uint16_t quantizer{};
  std::uint32_t n{};
  std::uint32_t k{};
  std::uint32_t padded_n{};
  std::uint32_t padded_k{};
  std::uint64_t codes_bytes{};
  std::uint64_t scales_bytes{};
};

enum class PrefillEpilogue : std::uint8_t {
  StoreBf16 = 1,
  StoreFp32 = 2,
  ResidualAddFp32 = 3,
};

enum class PrefillDispatch : std::uint8_t {
  BoundedUnpackBf16Cublas = 1,
  LocalQ4K = 2,
};

// Token-major device arrays; output has stride weight.n and only valid_tokens
// rows are written. first_position is the caller's absolute token range.
struct PrefillProjection {
  PrefillWeight weight{};
  std::uint16_t const* input{};
  void* output{};
  float const* residual{};
  std::uint32_t valid_tokens{};
  std::uint64_t first_position{};
  PrefillEpilogue epilogue{PrefillEpilogue::StoreBf16};
  Fp8Input packed{};
};

class PrefillEngine {
 public:
  // The Stream and every borrowed buffer outlive the engine and its work.
  PrefillEngine() = default;
  PrefillEngine(PrefillEngine&& other) noexcept;
  PrefillEngine& operator=(PrefillEngine&& other) noexcept;
  ~PrefillEngine();
  PrefillEngine(PrefillEngine const&) = delete;
  PrefillEngine& operator=(PrefillEngine const&) = delete;

  // Both dispatch policies run the same BF16 MFMA projection here; fp8 = true
  // is rejected (no FP8 path on this build).
  [[nodiscard]] static expected<PrefillEngine, Error> create(
      Stream const& stream, std::uint32_t token_capacity = kPrefillDefaultTokens,
      std::uint32_t weight_rows = kPrefillDefaultWeightRows,
      PrefillDispatch dispatch = PrefillDispatch::BoundedUnpackBf16Cublas, bool fp8 = false);

  [[nodiscard]] Fp8Input fp8_operand(unsigned m, unsigned k) const noexcept;
  [[nodiscard]] expected<void, Error> project(PrefillProjection const& projection);
  [[nodiscard]] expected<void, Error> paired_swiglu(PrefillWeight const& gate,
                                                         PrefillWeight const& up,
                                                         std::uint16_t const* normalized,
                                                         std::uint16_t* swiglu,
                                                         std::uint32_t valid_tokens,
                                                         std::uint64_t first_position);
  [[nodiscard]] expected<void, Error> mlp(PrefillWeight const& gate, PrefillWeight const& up,
                                               PrefillWeight const& down, float const* h_mid,
                                               std::uint16_t const* gamma, float eps,
                                               float* next_h, std::uint32_t valid_tokens,
                                               std::uint64_t first_position);
  // Vocabulary head (248320 x 5120): generation reads the final row,
  // evaluation the requested rows in caller order (at most eight).
  [[nodiscard]] expected<void, Error> head_generation(PrefillWeight const& head,
                                                           std::uint16_t const* normalized,
                                                           std::uint32_t valid_tokens,
                                                           std::uint64_t first_position,
                                                           float* logits);
  [[nodiscard]] expected<void, Error> head_evaluation(
      PrefillWeight const& head, std::uint16_t const* normalized, std::uint32_t valid_tokens,
      std::uint64_t first_position, std::span<std::uint32_t const> requested_rows, float* logits);

  [[nodiscard]] std::uint64_t workspace_bytes() const noexcept { return workspace_.bytes(); }
  [[nodiscard]] std::uint32_t token_capacity() const noexcept { return token_capacity_; }
  [[nodiscard]] std::uint32_t weight_rows() const noexcept { return weight_rows_; }
  [[nodiscard]] Stream const* stream() const noexcept { return stream_; }

 private:
  [[nodiscard]] expected<void, Error> ready(char const* op) const;

  Stream const* stream_{};
  hipStream_t native_stream_{};
  int device_{-1};
  DeviceBuffer workspace_{};  // normalized BF16 + SwiGLU BF16 slabs of the MLP
  std::uint32_t token_capacity_{};
  std::uint32_t weight_rows_{};
  PrefillDispatch dispatch_{PrefillDispatch::BoundedUnpackBf16Cublas};
};

}  // namespace qw38::cuda
