// Runtime callers of the Q8 projection path (interface subset of
// runtime/mlp.hpp, runtime/prefill.hpp and the decode-token graph of
// runtime/language_model.cpp in Enucatl/qw38): an MLP plan bound from an
// uploaded Model and a Session, its submission (Q8 MLP through q4k_q8_mlp with
// the session workspace, or the BF16 decode_mmv / PrefillEngine route), and
// a captured decode token replayed per token.
#pragma once

#include <cstdint>
#include <span>

#include "cuda/buffer.hpp"
#include "cuda/graph.hpp"
#include "cuda/prefill.hpp"
#include "cuda/stream.hpp"
#include "runtime/model.hpp"

namespace qw38::runtime {

inline constexpr std::uint32_t kHidden = 5120;      // runtime/sizes.hpp:38
inline constexpr std::uint32_t kFfnWidth = 17408;   // runtime/sizes.hpp:39
inline constexpr float kMlpRmsEps = 1.0e-6f;        // runtime/mlp.hpp:19

// A submission that failed after device work started poisons its session
// (runtime/session.hpp): later submissions are rejected.
class SessionExecutionState {
 public:
  void poison() noexcept { poisoned_ = true; }
  [[nodiscard]] bool is_poisoned() const noexcept { return poisoned_; }

 private:
  bool poisoned_{};
};

// Per-session device state the MLP needs: the Q8 MLP workspace for up to
// `q8_tokens` tokens (cuda::q8_mlp_workspace_bytes), owned for the session.
class Session {
 public:
  [[nodiscard]] static expected<Session, Error> create(cuda::Stream const& stream, std::uint32_t q8_tokens);
  [[nodiscard]] std::span<std::byte> q8_mlp_workspace() noexcept {
    return {workspace_.as_bytes(), std::size_t(workspace_.bytes())};
  }
  [[nodiscard]] SessionExecutionState& state() noexcept { return state_; }

 private:
  cuda::DeviceBuffer workspace_;
  SessionExecutionState state_;
};

// Activation buffers of one MLP invocation (device memory owned by the caller).
struct MlpBuffers {
  float const* h_mid{};          // FP32 [m][5120], preserved through the down add
  float* next_h{};               // FP32 [m][5120] = h_mid + down projection
  std::uint16_t* normalized{};   // BF16 [5120] (BF16 decode route)
  std::uint16_t* swiglu{};       // BF16 [17408] (BF16 decode route)
};

enum class MlpRoute : std::uint8_t { Q8, Bf16 };

struct MlpPlan {
  cuda::PrefillWeight gate{}, up{}, down{};
  std::uint16_t const* gamma{};
  MlpBuffers io{};
  cuda::Stream const* stream{};
  SessionExecutionState* session_state{};
  float eps{kMlpRmsEps};
  MlpRoute route{MlpRoute::Q8};
  std::span<std::byte> q8_workspace{};
};

// Resolves model.language_model.layers.<layer>.mlp.{gate,up,down}_proj.weight
// and .post_attention_layernorm.weight (runtime/mlp.cpp:392-411), checks the
// 5120 <-> 17408 geometry and binds the session's Q8 workspace (Q8 route).
[[nodiscard]] expected<MlpPlan, Error> bind_mlp_plan(Model const& model, Session& session,
                                                     std::uint32_t layer, cuda::Stream const& stream,
                                                     MlpBuffers const& io, MlpRoute route = MlpRoute::Q8,
                                                     float eps = kMlpRmsEps);

namespace detail {
struct Submission {
  // Enqueues one decode-token MLP (m = 1) on plan.stream; with `failure` non-null
  // the nonfinite-producer flag stays on the device (graph capture), otherwise
  // the Q8 route completes and reports it (runtime/mlp.cpp:597-669).
  [[nodiscard]] static expected<void, Error> mlp(MlpPlan const& plan, int* failure);
  // Prefill chunk of `tokens` tokens: Q8 route through q4k_q8_mlp with the
  // session workspace, BF16 route through PrefillEngine::mlp
  // (runtime/prefill.cpp:235-258).
  [[nodiscard]] static expected<void, Error> prefill_mlp(MlpPlan const& plan, cuda::PrefillEngine& engine,
                                                         float const* h_mid, float* next_h,
                                                         std::uint32_t tokens, std::uint64_t first_position,
                                                         int* failure);
};
}  // namespace detail

// Public synchronous entry points reject a capturing stream.
[[nodiscard]] expected<void, Error> execute_decode_mlp(MlpPlan const& plan);
[[nodiscard]] expected<void, Error> execute_prefill_mlp(MlpPlan const& plan, cuda::PrefillEngine& engine,
                                                        float const* h_mid, float* next_h,
                                                        std::uint32_t tokens, std::uint64_t first_position);

// One decode token's MLP captured into a hipGraph and replayed per token
// (runtime/language_model.cpp:324-330: capture at a token boundary, replay,
// then complete_unit reads the device failure flag back and waits). The flag
// is cleared by a captured fill kernel at the start of every replay.
class DecodeMlpGraph {
 public:
  [[nodiscard]] static expected<DecodeMlpGraph, Error> capture(MlpPlan const& plan);
  [[nodiscard]] expected<void, Error> launch() const;
  [[nodiscard]] expected<void, Error> complete_unit() const;

 private:
  MlpPlan plan_{};
  cuda::DeviceBuffer failure_;
  cuda::Graph graph_;
};

}  // namespace qw38::runtime
