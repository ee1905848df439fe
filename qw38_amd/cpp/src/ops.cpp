// qw38::cuda operators of the projection path over the C-ABI of libqw38_hip:
// q4k_q8 (cuda/q4k_q8.hpp), the hidden RMS producers (cuda/activation.hpp),
// decode_mmv (cuda/decode_mmv.hpp), the FP8 entry points (cuda/fp8.hpp, not
// implemented) and the BF16 PrefillEngine (cuda/prefill.hpp).
#include <hip/hip_runtime.h>

#include <cmath>
#include <limits>
#include <utility>
#include <vector>

#include "cuda/activation.hpp"
#include "cuda/decode_mmv.hpp"
#include "cuda/fp8.hpp"
#include "cuda/graph.hpp"
#include "cuda/prefill.hpp"
#include "cuda/q4k_q8.hpp"
#include "qw38_hip.h"

namespace qw38::cuda {
namespace {

qw38_weight abi(PrefillWeight const& w) {
  return qw38_weight{w.codes, w.scales, w.layout, w.quantizer, w.n, w.k,
                     w.padded_n, w.padded_k, w.codes_bytes, w.scales_bytes};
}

qw38_q8_input abi(Q8Input const& q) {
  return qw38_q8_input{q.codes.data(), q.codes.size(), q.scales.data(), q.scales.size(),
                       q.sums.data(), q.sums.size(), q.m, q.k, q.padded_k};
}

qw38_decode_view abi(DecodeOperandView const& v) {
  qw38_decode_view r{};
  r.pointer = v.pointer;
  r.space = static_cast<uint8_t>(v.space);
  r.dtype = static_cast<uint8_t>(v.dtype);
  r.layout = v.layout;
  r.logical_n = v.logical_n;
  r.logical_k = v.logical_k;
  r.padded_n = v.padded_n;
  r.padded_k = v.padded_k;
  r.bytes = v.bytes;
  r.alignment = v.alignment;
  r.writable = v.writable ? 1 : 0;
  // An empty reference view (default member values) maps to an all-zero view.
  if (v == DecodeOperandView{}) r = qw38_decode_view{};
  return r;
}

qw38_decode_desc abi(DecodeMmvDesc const& d) {
  qw38_decode_desc r{};
  r.layout = d.layout;
  r.quantizer = d.quantizer;
  r.activation_policy = static_cast<uint8_t>(d.activation_policy);
  r.n = d.n;
  r.k = d.k;
  r.padded_n = d.padded_n;
  r.padded_k = d.padded_k;
  r.codes = abi(d.codes);
  r.scales = abi(d.scales);
  r.input = abi(d.input);
  r.output = abi(d.output);
  r.residual = abi(d.residual);
  r.epilogue = static_cast<uint8_t>(d.epilogue);
  return r;
}

expected<void, Error> require_stream(Stream const& stream, char const* op) {
  if (stream.empty()) return unexpected(make_error(ErrorCode::InvalidArgument, op, "empty stream"));
  return {};
}

Error not_implemented(char const* op, char const* what) {
  return make_error(ErrorCode::InvalidArgument, op, std::string(what) + " is not implemented on this build");
}

}  // namespace

// ---- q4k_q8 -----------------------------------------------------------------------
expected<void, Error> pack_q8(std::span<std::uint16_t const> input, Q8Input output,
                              std::span<int> failure, Stream const& stream) {
  if (auto st = require_stream(stream, "q8.pack"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const qw38_q8_input q = abi(output);
  return from_abi(qw38_pack_q8(input.data(), input.size(), &q, failure.data(), failure.size(),
                               stream.native()));
}

expected<void, Error> q4k_q8_project(PrefillWeight const& weight, Q8Input input,
                                     std::span<float> output, Stream const& stream,
                                     std::span<float const> residual) {
  if (auto st = require_stream(stream, "q8.project"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const qw38_weight w = abi(weight);
  const qw38_q8_input q = abi(input);
  return from_abi(qw38_q4k_q8_project(&w, &q, output.data(), output.size(),
                                      residual.empty() ? nullptr : residual.data(), residual.size(),
                                      stream.native()));
}

expected<void, Error> q4k_q8_mlp(PrefillWeight const& gate, PrefillWeight const& up,
                                 PrefillWeight const& down, float const* residual,
                                 std::uint16_t const* gamma, float eps, float* output, unsigned m,
                                 std::span<std::byte> workspace, Stream const& stream,
                                 bool& submitted, int* pending_failure) {
  submitted = false;
  if (auto st = require_stream(stream, "q8.mlp"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const qw38_weight g = abi(gate), u = abi(up), d = abi(down);
  int sub = 0;
  auto r = from_abi(qw38_q4k_q8_mlp(&g, &u, &d, residual, gamma, eps, output, m, workspace.data(),
                                    workspace.size(), stream.native(), &sub, pending_failure));
  submitted = sub != 0;
  return r;
}

// ---- hidden RMS producers ---------------------------------------------------------
expected<void, Error> launch_hidden_rms_q8(float const* residual, std::uint16_t const* gamma,
                                           float eps, unsigned m, std::int8_t* codes,
                                           float* scales, std::int32_t* sums, int* failure,
                                           Stream const& stream) {
  if (auto st = require_stream(stream, "hidden_rms_q8"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return from_abi(qw38_hidden_rms_q8(residual, gamma, eps, m, codes, scales, sums, failure,
                                     stream.native()));
}

expected<void, Error> launch_hidden_rms(float const* residual, std::uint16_t const* gamma, float eps,
                                        std::uint32_t n_tokens, std::uint16_t* out_bf16,
                                        Stream const& stream) {
  if (auto st = require_stream(stream, "hidden_rms"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return from_abi(qw38_hidden_rms_bf16(residual, gamma, eps, n_tokens, out_bf16, stream.native()));
}

// ---- decode_mmv -------------------------------------------------------------------
expected<void, Error> launch_decode_mmv(DecodeMmvDesc const& desc, Stream const& stream) {
  if (auto st = require_stream(stream, "decode_mmv"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const qw38_decode_desc d = abi(desc);
  return from_abi(qw38_decode_mmv(&d, stream.native()));
}

expected<void, Error> launch_decode_mmv_paired(DecodeMmvPairedDesc const& desc, Stream const& stream) {
  if (auto st = require_stream(stream, "decode_mmv_paired"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const qw38_decode_desc a = abi(desc.a), b = abi(desc.b);
  return from_abi(qw38_decode_mmv_paired(&a, &b, stream.native()));
}

expected<void, Error> launch_decode_ab_bf16(DecodeMmvPairedDesc const& desc, Stream const& stream) {
  if (auto st = require_stream(stream, "decode_ab_bf16"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const qw38_decode_desc a = abi(desc.a), b = abi(desc.b);
  return from_abi(qw38_decode_ab_bf16(&a, &b, stream.native()));
}

expected<void, Error> launch_decode_mmv_ranges(DecodeMmvRangeDesc const& desc, Stream const& stream) {
  if (auto st = require_stream(stream, "decode_mmv_ranges"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  std::vector<qw38_decode_desc> ds;
  ds.reserve(desc.ranges.size());
  for (auto const& d : desc.ranges) ds.push_back(abi(d));
  return from_abi(qw38_decode_mmv_ranges(ds.data(), uint32_t(ds.size()), stream.native()));
}

// ---- FP8 (types only on this build) -------------------------------------------------
expected<void, Error> pack_fp8(std::span<std::uint16_t const>, unsigned, unsigned,
                               std::span<std::uint8_t>, std::span<float>, Stream const&) {
  return unexpected(not_implemented("fp8.pack", "FP8"));
}

expected<void, Error> fp8_gemv(Fp8Weight, std::span<std::uint16_t const>, std::span<float>,
                               Stream const&) {
  return unexpected(not_implemented("fp8.gemv", "FP8"));
}

// ---- PrefillEngine ---------------------------------------------------------------
expected<void, Error> validate_prefill_device_span(void const* pointer, std::uint64_t bytes,
                                                   std::uint32_t alignment, int device) {
  constexpr char const* op = "prefill.span";
  if (!pointer || !bytes || !alignment || (alignment & (alignment - 1)) ||
      reinterpret_cast<std::uintptr_t>(pointer) % alignment)
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "null, empty or misaligned span"));
  const auto b = reinterpret_cast<std::uintptr_t>(pointer);
  if (bytes > std::numeric_limits<std::uintptr_t>::max() - b)
    return unexpected(make_error(ErrorCode::Overflow, op, "address overflow"));
  hipPointerAttribute_t attr{};
  if (hipPointerGetAttributes(&attr, pointer) != hipSuccess) {
    (void)hipGetLastError();
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "span is not device memory"));
  }
  if (attr.type != hipMemoryTypeDevice || attr.device != device)
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "span is not memory of the device"));
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(pointer)) != hipSuccess) {
    (void)hipGetLastError();
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "allocation range unknown"));
  }
  const auto lo = reinterpret_cast<std::uintptr_t>(base);
  if (b < lo || b + bytes > lo + size)
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "span exceeds its allocation"));
  return {};
}

PrefillEngine::PrefillEngine(PrefillEngine&& other) noexcept { *this = std::move(other); }

PrefillEngine& PrefillEngine::operator=(PrefillEngine&& other) noexcept {
  if (this != &other) {
    stream_ = std::exchange(other.stream_, nullptr);
    native_stream_ = std::exchange(other.native_stream_, nullptr);
    device_ = std::exchange(other.device_, -1);
    workspace_ = std::move(other.workspace_);
    token_capacity_ = std::exchange(other.token_capacity_, 0);
    weight_rows_ = std::exchange(other.weight_rows_, 0);
    dispatch_ = other.dispatch_;
  }
  return *this;
}

PrefillEngine::~PrefillEngine() = default;

expected<PrefillEngine, Error> PrefillEngine::create(Stream const& stream,
                                                     std::uint32_t token_capacity,
                                                     std::uint32_t weight_rows,
                                                     PrefillDispatch dispatch, bool fp8) {
  if (stream.empty() || token_capacity == 0 || token_capacity > kPrefillMaxTokens ||
      (weight_rows != 128 && weight_rows != 256 && weight_rows != 512) ||
      (dispatch != PrefillDispatch::BoundedUnpackBf16Cublas && dispatch != PrefillDispatch::LocalQ4K))
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.create",
                                 "invalid stream or token capacity"));
  if (fp8) return unexpected(not_implemented("prefill.create", "the FP8 prefill path"));
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  auto buffer = DeviceBuffer::allocate(qw38_prefill_mlp_workspace_bytes(token_capacity), stream.device());
  if (!buffer) return unexpected(buffer.error());
  PrefillEngine e;
  e.stream_ = &stream;
  e.native_stream_ = stream.native();
  e.device_ = stream.device();
  e.workspace_ = std::move(*buffer);
  e.token_capacity_ = token_capacity;
  e.weight_rows_ = weight_rows;
  e.dispatch_ = dispatch;
  return e;
}

expected<void, Error> PrefillEngine::ready(char const* op) const {
  if (!stream_ || stream_->empty() || stream_->native() != native_stream_ ||
      stream_->device() != device_ || workspace_.empty())
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "stream is closed"));
  return {};
}

Fp8Input PrefillEngine::fp8_operand(unsigned, unsigned) const noexcept { return {}; }

expected<void, Error> PrefillEngine::project(PrefillProjection const& d) {
  if (auto st = ready("prefill.project"); !st) return st;
  auto guard = stream_->activate();
  if (!guard) return unexpected(guard.error());
  if (d.valid_tokens == 0 || d.valid_tokens > token_capacity_)
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.weight",
                                 "weight, layout or token contract mismatch"));
  if (!d.input || !d.output ||
      d.first_position > std::numeric_limits<std::uint64_t>::max() - d.valid_tokens)
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.project",
                                 "input, output, position or epilogue contract mismatch"));
  const qw38_weight w = abi(d.weight);
  return from_abi(qw38_prefill_project(&w, d.input, d.valid_tokens, d.output, d.residual,
                                       static_cast<int>(d.epilogue), native_stream_));
}

expected<void, Error> PrefillEngine::paired_swiglu(PrefillWeight const& gate, PrefillWeight const& up,
                                                   std::uint16_t const* normalized,
                                                   std::uint16_t* swiglu, std::uint32_t valid_tokens,
                                                   std::uint64_t first_position) {
  if (auto st = ready("prefill.swiglu"); !st) return st;
  auto guard = stream_->activate();
  if (!guard) return unexpected(guard.error());
  if (valid_tokens == 0 || valid_tokens > token_capacity_ ||
      first_position > std::numeric_limits<std::uint64_t>::max() - valid_tokens)
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.swiglu",
                                 "paired weight or activation contract mismatch"));
  const qw38_weight g = abi(gate), u = abi(up);
  return from_abi(qw38_prefill_paired_swiglu(&g, &u, normalized, swiglu, valid_tokens, native_stream_));
}

expected<void, Error> PrefillEngine::mlp(PrefillWeight const& gate, PrefillWeight const& up,
                                         PrefillWeight const& down, float const* h_mid,
                                         std::uint16_t const* gamma, float eps, float* next_h,
                                         std::uint32_t valid_tokens, std::uint64_t first_position) {
  if (auto st = ready("prefill.mlp"); !st) return st;
  auto guard = stream_->activate();
  if (!guard) return unexpected(guard.error());
  if (valid_tokens == 0 || valid_tokens > token_capacity_ ||
      first_position > std::numeric_limits<std::uint64_t>::max() - valid_tokens)
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.mlp",
                                 "MLP shape or pointer contract mismatch"));
  const qw38_weight g = abi(gate), u = abi(up), dn = abi(down);
  return from_abi(qw38_prefill_mlp(&g, &u, &dn, h_mid, gamma, eps, next_h, valid_tokens,
                                   workspace_.as_bytes(), workspace_.bytes(), native_stream_));
}

expected<void, Error> PrefillEngine::head_generation(PrefillWeight const& head,
                                                     std::uint16_t const* normalized,
                                                     std::uint32_t valid_tokens,
                                                     std::uint64_t first_position, float* logits) {
  if (!normalized || !logits || valid_tokens == 0 || valid_tokens > token_capacity_ ||
      head.n != 248320 || head.k != 5120 ||
      first_position > std::numeric_limits<std::uint64_t>::max() - valid_tokens)
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.head",
                                 "generation head contract mismatch"));
  return project(PrefillProjection{.weight = head,
                                   .input = normalized + std::uint64_t(valid_tokens - 1u) * head.k,
                                   .output = logits,
                                   .valid_tokens = 1,
                                   .first_position = first_position + valid_tokens - 1u,
                                   .epilogue = PrefillEpilogue::StoreFp32});
}

expected<void, Error> PrefillEngine::head_evaluation(PrefillWeight const& head,
                                                     std::uint16_t const* normalized,
                                                     std::uint32_t valid_tokens,
                                                     std::uint64_t first_position,
                                                     std::span<std::uint32_t const> requested_rows,
                                                     float* logits) {
  if (!normalized || !logits || requested_rows.empty() || requested_rows.size() > kPrefillHeadRows ||
      head.n != 248320 || head.k != 5120 || valid_tokens == 0 || valid_tokens > token_capacity_ ||
      first_position > std::numeric_limits<std::uint64_t>::max() - valid_tokens)
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.head",
                                 "evaluation head contract mismatch"));
  for (std::size_t i = 0; i < requested_rows.size(); ++i) {
    if (requested_rows[i] >= valid_tokens)
      return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.head.rows",
                                   "requested row is out of range"));
    for (std::size_t j = 0; j < i; ++j)
      if (requested_rows[i] == requested_rows[j])
        return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.head.rows",
                                     "duplicate requested row"));
  }
  for (std::size_t i = 0; i < requested_rows.size(); ++i) {
    const auto row = requested_rows[i];
    if (auto st = project(PrefillProjection{.weight = head,
                                            .input = normalized + std::uint64_t(row) * head.k,
                                            .output = logits + std::uint64_t(i) * head.n,
                                            .valid_tokens = 1,
                                            .first_position = first_position + row,
                                            .epilogue = PrefillEpilogue::StoreFp32});
        !st)
      return st;
  }
  return {};
}

}  // namespace qw38::cuda
