// Prefill engine (interface of cuda/prefill.hpp in Enucatl/qw38). Q4_K 0x020D
// weights run on this build's BF16 MFMA projection (the Q8 MMQ path is
// q4k_q8_project); FP8 0x020F weights run on the FP8 GEMM with a fused
// epilogue (M > 1) or decode_mmv (M = 1). Other layouts are rejected.
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
inline constexpr std::uint32_t kFp8MaxK = 6144;  // FP8 prefill projections: k <= 6144

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
  Fp8Input packed{};  // FP8 with M > 1: fp8_operand(valid_tokens, k), packed by the caller
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
  // also reserves the engine-owned FP8 activation operand (codes + scales of
  // up to token_capacity x 6144).
  [[nodiscard]] static expected<PrefillEngine, Error> create(
      Stream const& stream, std::uint32_t token_capacity = kPrefillDefaultTokens,
      std::uint32_t weight_rows = kPrefillDefaultWeightRows,
      PrefillDispatch dispatch = PrefillDispatch::BoundedUnpackBf16Cublas, bool fp8 = false);

  // The engine-owned operand for pack_fp8 of m tokens of width k (k <= 6144,
  // k % 128 == 0); empty without an FP8 engine or for an invalid shape.
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

  [[nodiscard]] std::uint64_t workspace_bytes() const noexcept {
    return workspace_.bytes() + fp8_workspace_.bytes();
  }
  [[nodiscard]] std::uint32_t token_capacity() const noexcept { return token_capacity_; }
  [[nodiscard]] std::uint32_t weight_rows() const noexcept { return weight_rows_; }
  [[nodiscard]] Stream const* stream() const noexcept { return stream_; }

 private:
  [[nodiscard]] expected<void, Error> ready(char const* op) const;
  [[nodiscard]] expected<void, Error> project_fp8(PrefillProjection const& projection);
  // NVFP4 scratch: the region after the MLP slabs of workspace_.
  [[nodiscard]] void* nvfp4_scratch() const noexcept;
  [[nodiscard]] std::uint64_t nvfp4_scratch_bytes() const noexcept;

  Stream const* stream_{};
  hipStream_t native_stream_{};
  int device_{-1};
  DeviceBuffer workspace_{};  // normalized BF16 + SwiGLU BF16 slabs of the MLP
  std::uint32_t token_capacity_{};
  std::uint32_t weight_rows_{};
  PrefillDispatch dispatch_{PrefillDispatch::BoundedUnpackBf16Cublas};
  DeviceBuffer fp8_workspace_{};  // FP8 operand: codes [cap][6144], scales [48][cap]
  int fp8_sm_count_{};
};

}  // namespace qw38::cuda
