// Runtime MLP submission over the Q8 projection path (runtime/mlp.cpp:560-669,
// runtime/prefill.cpp:235-258 and the decode-token graph of
// runtime/language_model.cpp:324-330 in Enucatl/qw38 define the callers this
// file mirrors).
#include "runtime/mlp.hpp"

#include <string>

#include "cuda/activation.hpp"
#include "cuda/decode_mmv.hpp"
#include "cuda/error.hpp"
#include "cuda/q4k_q8.hpp"
#include "cuda/stream.hpp"

namespace qw38::runtime {
namespace {

Error arg_error(std::string_view op, std::string_view detail) {
  return cuda::make_error(cuda::ErrorCode::InvalidArgument, op, detail);
}

std::string layer_name(std::uint32_t layer, char const* suffix) {
  return "model.language_model.layers." + std::to_string(layer) + suffix;
}

// Q4_K 0x020D weight as a BF16-input decode_mmv descriptor (runtime/mlp.cpp
// mmv_from_weight): the same tiles feed the BF16 decode route.
cuda::DecodeMmvDesc mmv_from_weight(cuda::PrefillWeight const& w) {
  cuda::DecodeMmvDesc d;
  d.layout = w.layout;
  d.quantizer = w.quantizer;
  d.n = w.n;
  d.k = w.k;
  d.padded_n = w.padded_n;
  d.padded_k = w.padded_k;
  d.codes = cuda::decode_matrix_view(const_cast<void*>(w.codes), cuda::DecodeDtype::Q4, w.layout, w.n, w.k,
                                     w.padded_n, w.padded_k, w.codes_bytes, 16);
  // scales: [padded_n][padded_k / 256 super-blocks][8 fp16] per the 0x020D contract
  const std::uint32_t units = w.padded_k / 256u * 8u;
  d.scales = cuda::decode_matrix_view(const_cast<void*>(w.scales), cuda::DecodeDtype::Fp16, w.layout,
                                      w.padded_n, units, w.padded_n, units, w.scales_bytes, 2);
  return d;
}

}  // namespace

expected<Session, Error> Session::create(cuda::Stream const& stream, std::uint32_t q8_tokens) {
  if (!q8_tokens || q8_tokens > QW38_Q8_MLP_MAX_TOKENS)
    return cuda::unexpected(arg_error("session", "Q8 MLP token capacity must be 1..512"));
  auto ws = cuda::DeviceBuffer::allocate(cuda::q8_mlp_workspace_bytes(q8_tokens), stream.device());
  if (!ws) return cuda::unexpected(ws.error());
  Session s;
  s.workspace_ = std::move(*ws);
  return s;
}

expected<MlpPlan, Error> bind_mlp_plan(Model const& model, Session& session, std::uint32_t layer,
                                       cuda::Stream const& stream, MlpBuffers const& io, MlpRoute route,
                                       float eps) {
  MlpPlan plan;
  auto gate = model.weight(layer_name(layer, ".mlp.gate_proj.weight"));
  auto up = model.weight(layer_name(layer, ".mlp.up_proj.weight"));
  auto down = model.weight(layer_name(layer, ".mlp.down_proj.weight"));
  auto gamma = model.payload(layer_name(layer, ".post_attention_layernorm.weight"));
  if (!gate) return cuda::unexpected(gate.error());
  if (!up) return cuda::unexpected(up.error());
  if (!down) return cuda::unexpected(down.error());
  if (!gamma) return cuda::unexpected(gamma.error());
  if (gate->n != kFfnWidth || gate->k != kHidden || up->n != kFfnWidth || up->k != kHidden ||
      down->n != kHidden || down->k != kFfnWidth || gamma->bytes != kHidden * 2)
    return cuda::unexpected(arg_error("mlp.bind", "MLP weights must be 5120 -> 17408 -> 5120"));
  if (route == MlpRoute::Bf16 &&
      (gate->layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 || up->layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 ||
       down->layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 || !io.normalized || !io.swiglu))
    return cuda::unexpected(arg_error("mlp.bind", "BF16 route needs 0x020D weights and BF16 scratch views"));
  if (!io.h_mid || !io.next_h) return cuda::unexpected(arg_error("mlp.bind", "null h_mid / next_h"));
  plan.gate = *gate;
  plan.up = *up;
  plan.down = *down;
  plan.gamma = static_cast<std::uint16_t const*>(gamma->pointer);
  plan.io = io;
  plan.stream = &stream;
  plan.session_state = &session.state();
  plan.eps = eps;
  plan.route = route;
  if (route == MlpRoute::Q8) {
    plan.q8_workspace = session.q8_mlp_workspace();
    if (plan.q8_workspace.size() < cuda::q8_mlp_workspace_bytes(1))
      return cuda::unexpected(arg_error("q8.workspace", "missing session Q8 MLP workspace"));
  }
  return plan;
}

expected<void, Error> detail::Submission::mlp(MlpPlan const& plan, int* failure) {
  if (plan.session_state && plan.session_state->is_poisoned())
    return cuda::unexpected(arg_error("session", "session is poisoned"));
  if (!plan.stream || plan.stream->empty()) return cuda::unexpected(arg_error("stream", "empty stream"));
  auto const& s = *plan.stream;
  if (plan.route == MlpRoute::Q8) {
    bool submitted = false;
    auto st = cuda::q4k_q8_mlp(plan.gate, plan.up, plan.down, plan.io.h_mid, plan.gamma, plan.eps,
                               plan.io.next_h, 1, plan.q8_workspace, s, submitted, failure);
    if (!st) {
      if (submitted && plan.session_state) plan.session_state->poison();
      return cuda::unexpected(st.error());
    }
    return {};
  }
  // BF16 route: RMS -> BF16, paired gate/up with the SwiGLU BF16 epilogue,
  // down with the FP32 residual add.
  if (auto st = cuda::launch_hidden_rms(plan.io.h_mid, plan.gamma, plan.eps, 1, plan.io.normalized, s); !st)
    return cuda::unexpected(st.error());
  cuda::DecodeMmvPairedDesc paired;
  paired.a = mmv_from_weight(plan.gate);
  paired.a.input = cuda::decode_vector_view(plan.io.normalized, cuda::DecodeDtype::Bf16,
                                            cuda::kDecodeLayoutBf16VectorV0, kHidden, kHidden * 2u, 2, false);
  paired.a.output = cuda::decode_vector_view(plan.io.swiglu, cuda::DecodeDtype::Bf16,
                                             cuda::kDecodeLayoutBf16VectorV0, kFfnWidth, kFfnWidth * 2u, 2, true);
  paired.a.epilogue = cuda::DecodeEpilogue::SwigluStoreBf16;
  paired.b = mmv_from_weight(plan.up);
  paired.b.input = paired.a.input;
  paired.b.epilogue = paired.a.epilogue;
  if (auto st = cuda::launch_decode_mmv_paired(paired, s); !st) return cuda::unexpected(st.error());
  cuda::DecodeMmvDesc down = mmv_from_weight(plan.down);
  down.input = cuda::decode_vector_view(plan.io.swiglu, cuda::DecodeDtype::Bf16, cuda::kDecodeLayoutBf16VectorV0,
                                        kFfnWidth, kFfnWidth * 2u, 2, false);
  down.residual = cuda::decode_vector_view(const_cast<float*>(plan.io.h_mid), cuda::DecodeDtype::Fp32,
                                           cuda::kDecodeLayoutFp32VectorV0, kHidden, kHidden * 4u, 4, false);
  down.output = cuda::decode_vector_view(plan.io.next_h, cuda::DecodeDtype::Fp32, cuda::kDecodeLayoutFp32VectorV0,
                                         kHidden, kHidden * 4u, 4, true);
  down.epilogue = cuda::DecodeEpilogue::ResidualAddFp32;
  if (auto st = cuda::launch_decode_mmv(down, s); !st) return cuda::unexpected(st.error());
  return {};
}

expected<void, Error> detail::Submission::prefill_mlp(MlpPlan const& plan, cuda::PrefillEngine& engine,
                                                      float const* h_mid, float* next_h, std::uint32_t tokens,
                                                      std::uint64_t first_position, int* failure) {
  if (plan.session_state && plan.session_state->is_poisoned())
    return cuda::unexpected(arg_error("session", "session is poisoned"));
  if (plan.route == MlpRoute::Q8) {
    if (engine.stream() != plan.stream || !tokens || tokens > engine.token_capacity() ||
        first_position > UINT64_MAX - tokens ||
        plan.q8_workspace.size() < cuda::q8_mlp_workspace_bytes(tokens))
      return cuda::unexpected(arg_error("q8.prefill", "invalid engine or token range"));
    bool submitted = false;
    auto st = cuda::q4k_q8_mlp(plan.gate, plan.up, plan.down, h_mid, plan.gamma, plan.eps, next_h, tokens,
                               plan.q8_workspace, *engine.stream(), submitted, failure);
    if (!st) {
      if (submitted && plan.session_state) plan.session_state->poison();
      return cuda::unexpected(st.error());
    }
    return {};
  }
  auto st = engine.mlp(plan.gate, plan.up, plan.down, h_mid, plan.gamma, plan.eps, next_h, tokens,
                       first_position);
  if (!st) return cuda::unexpected(st.error());
  return {};
}

expected<void, Error> execute_decode_mlp(MlpPlan const& plan) {
  if (plan.stream)
    if (auto st = cuda::require_uncaptured(*plan.stream); !st) return cuda::unexpected(st.error());
  return detail::Submission::mlp(plan, nullptr);
}

expected<void, Error> execute_prefill_mlp(MlpPlan const& plan, cuda::PrefillEngine& engine, float const* h_mid,
                                          float* next_h, std::uint32_t tokens, std::uint64_t first_position) {
  if (engine.stream())
    if (auto st = cuda::require_uncaptured(*engine.stream()); !st) return cuda::unexpected(st.error());
  return detail::Submission::prefill_mlp(plan, engine, h_mid, next_h, tokens, first_position, nullptr);
}

expected<DecodeMlpGraph, Error> DecodeMlpGraph::capture(MlpPlan const& plan) {
  if (!plan.stream) return cuda::unexpected(arg_error("stream", "empty stream"));
  if (auto st = cuda::require_uncaptured(*plan.stream); !st) return cuda::unexpected(st.error());
  DecodeMlpGraph g;
  g.plan_ = plan;
  auto flag = cuda::DeviceBuffer::allocate(sizeof(int), plan.stream->device());
  if (!flag) return cuda::unexpected(flag.error());
  g.failure_ = std::move(*flag);
  auto graph = cuda::Graph::begin(*plan.stream);
  if (!graph) return cuda::unexpected(graph.error());
  // the captured token: clear the flag (a fill kernel, not a memset node),
  // then the MLP with the device-side failure flag
  auto st = cuda::zero(g.failure_, *plan.stream);
  expected<void, Error> sub = st ? detail::Submission::mlp(plan, static_cast<int*>(g.failure_.data()))
                                 : expected<void, Error>(cuda::unexpected(st.error()));
  auto fin = graph->finish();
  if (!sub) return cuda::unexpected(sub.error());
  if (!fin) return cuda::unexpected(fin.error());
  g.graph_ = std::move(*graph);
  return g;
}

expected<void, Error> DecodeMlpGraph::launch() const {
  if (plan_.session_state && plan_.session_state->is_poisoned())
    return cuda::unexpected(arg_error("session", "session is poisoned"));
  return graph_.launch(*plan_.stream);
}

expected<void, Error> DecodeMlpGraph::complete_unit() const {
  int host = 0;
  if (auto st = cuda::copy_d2h(&host, failure_.data(), sizeof(int), *plan_.stream); !st)
    return cuda::unexpected(st.error());
  if (auto st = plan_.stream->sync(); !st) return cuda::unexpected(st.error());
  if (host) {
    if (plan_.session_state) plan_.session_state->poison();
    return cuda::unexpected(arg_error("q8.producer", "nonfinite producer or invalid Q8 scale"));
  }
  return {};
}

}  // namespace qw38::runtime
