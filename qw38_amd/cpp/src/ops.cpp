// qw38::cuda operators of the projection path over the C-ABI of libqw38_hip:
// q4k_q8 (cuda/q4k_q8.hpp), the hidden RMS producers (cuda/activation.hpp),
// decode_mmv (cuda/decode_mmv.hpp), the FP8 entry points (cuda/fp8.hpp) and
// the PrefillEngine (cuda/prefill.hpp) with its BF16 and FP8 branches.
#include <hip/hip_runtime.h>

#include <cmath>
#include <limits>
#include <utility>
#include <vector>

#include "cuda/activation.hpp"
#include "cuda/decode_mmv.hpp"
#include "cuda/fp8.hpp"
#include "cuda/nvfp4.hpp"
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

// ---- FP8 (cuda/fp8.hpp) ------------------------------------------------------------
namespace {
qw38_fp8_weight abi(Fp8Weight const& w) {
  return qw38_fp8_weight{w.codes.data(), w.codes.size(), w.scales.data(), w.scales.size(), w.n, w.k};
}
qw38_fp8_input abi(Fp8Input const& x) {
  return qw38_fp8_input{x.codes.data(), x.codes.size(), x.scales.data(), x.scales.size(), x.m, x.k};
}
}  // namespace

expected<void, Error> fp8_decode(DecodeMmvDesc const& desc, Stream const& stream) {
  if (desc.layout != kDecodeLayoutFp8V1)
    return unexpected(make_error(ErrorCode::InvalidArgument, "fp8.decode", "not an FP8 descriptor"));
  return launch_decode_mmv(desc, stream);
}

expected<int, Error> prepare_fp8_gemm(Stream const& stream) {
  if (auto st = require_stream(stream, "fp8.prepare"); !st) return unexpected(st.error());
  int sm = 0;
  if (auto st = from_abi(qw38_fp8_prepare(stream.native(), &sm)); !st) return unexpected(st.error());
  return sm;
}

expected<void, Error> fp8_store_bf16(std::span<float const> input, std::span<std::uint16_t> output,
                                     Stream const& stream) {
  if (auto st = require_stream(stream, "fp8.store"); !st) return st;
  if (input.size() != output.size())
    return unexpected(make_error(ErrorCode::InvalidArgument, "fp8.v1", "invalid geometry, extent or alias"));
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return from_abi(qw38_fp8_store_bf16(input.data(), output.data(), input.size(), stream.native()));
}

expected<void, Error> pack_fp8(std::span<std::uint16_t const> input, unsigned m, unsigned k,
                               std::span<std::uint8_t> codes, std::span<float> scales,
                               Stream const& stream) {
  if (auto st = require_stream(stream, "fp8.pack"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return from_abi(qw38_pack_fp8(input.data(), input.size(), m, k, codes.data(), codes.size(),
                                scales.data(), scales.size(), stream.native()));
}

expected<void, Error> fp8_gemm(Fp8Weight weight, Fp8Input input, std::span<float> output,
                               std::span<std::byte> workspace, int sm_count, Stream const& stream) {
  if (auto st = require_stream(stream, "fp8.gemm"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const qw38_fp8_weight w = abi(weight);
  const qw38_fp8_input x = abi(input);
  return from_abi(qw38_fp8_gemm(&w, &x, output.data(), output.size(), workspace.data(),
                                workspace.size(), sm_count, stream.native()));
}

expected<void, Error> fp8_gemv(Fp8Weight weight, std::span<std::uint16_t const> input,
                               std::span<float> output, Stream const& stream) {
  if (auto st = require_stream(stream, "fp8.gemv"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const qw38_fp8_weight w = abi(weight);
  return from_abi(qw38_fp8_gemv(&w, input.data(), input.size(), output.data(), output.size(),
                                stream.native()));
}

// ---- NVFP4 (cuda/nvfp4.hpp) --------------------------------------------------------
namespace {
std::uint32_t pad256(std::uint32_t k) { return (k + 255u) / 256u * 256u; }
std::uint64_t pad128_rows(std::uint32_t m) { return (std::uint64_t(m) + 127u) / 128u * 128u; }
}  // namespace

expected<int, Error> prepare_nvfp4_gemm(std::uint32_t max_m, std::uint64_t workspace_bytes,
                                        Stream const& stream) {
  (void)workspace_bytes;
  if (auto st = require_stream(stream, "nvfp4.prepare"); !st) return unexpected(st.error());
  if (max_m == 0 || max_m > 1024)
    return unexpected(make_error(ErrorCode::InvalidArgument, "nvfp4.prepare", "invalid token capacity"));
  int sm = 0;
  if (auto st = from_abi(qw38_fp8_prepare(stream.native(), &sm)); !st) return unexpected(st.error());
  return sm;
}

expected<void, Error> nvfp4_gemm_tile(void const* codes, void const* scales,
                                      std::uint8_t const* activation,
                                      std::uint8_t const* activation_scales, std::uint32_t m,
                                      std::uint32_t n, std::uint32_t k, std::uint32_t row_start,
                                      float* output, void* workspace, std::uint64_t workspace_bytes,
                                      int sm_count, Stream const& stream) {
  (void)workspace;
  (void)workspace_bytes;
  (void)sm_count;
  if (auto st = require_stream(stream, "nvfp4.gemm"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return from_abi(qw38_nvfp4_gemm_tile(codes, scales, activation, activation_scales, m, n, k,
                                       row_start, output, stream.native()));
}

expected<void, Error> launch_pack_nvfp4(std::uint16_t const* input, std::uint8_t* codes,
                                        std::uint8_t* scales, std::uint32_t m, std::uint32_t k,
                                        Stream const& stream) {
  if (auto st = require_stream(stream, "nvfp4.pack"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const std::uint32_t pk = pad256(k);
  return from_abi(qw38_pack_nvfp4(input, m, k, codes, std::uint64_t(m) * (pk / 2), scales,
                                  pad128_rows(m) * (pk / 16), stream.native()));
}

expected<void, Error> launch_hidden_rms_fp8(float const* residual, std::uint16_t const* gamma,
                                            float eps, std::uint32_t n_tokens,
                                            std::uint16_t* companion, std::uint8_t* codes,
                                            float* scales, Stream const& stream) {
  if (auto st = require_stream(stream, "hidden_rms_fp8"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return from_abi(qw38_hidden_rms_fp8(residual, gamma, eps, n_tokens, companion, codes, scales,
                                      stream.native()));
}

expected<void, Error> launch_hidden_rms_nvfp4(float const* residual, std::uint16_t const* gamma,
                                              float eps, std::uint32_t n_tokens,
                                              std::uint8_t* codes, std::uint8_t* scales,
                                              Stream const& stream) {
  if (auto st = require_stream(stream, "hidden_rms_nvfp4"); !st) return st;
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return from_abi(qw38_hidden_rms_nvfp4(residual, gamma, eps, n_tokens, codes, scales,
                                        stream.native()));
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
    fp8_workspace_ = std::move(other.fp8_workspace_);
    fp8_sm_count_ = std::exchange(other.fp8_sm_count_, 0);
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
  if (fp8) {  // cuda/prefill.cu:424-430; no FP32 accumulator: the epilogue is fused
    auto sm = prepare_fp8_gemm(stream);
    if (!sm) return unexpected(sm.error());
    e.fp8_sm_count_ = *sm;
    const std::uint64_t cap = (token_capacity + 127) / 128 * 128;
    auto op = DeviceBuffer::allocate(cap * (kFp8MaxK + kFp8MaxK / 128 * 4), stream.device());
    if (!op) return unexpected(op.error());
    e.fp8_workspace_ = std::move(*op);
  }
  return e;
}

expected<void, Error> PrefillEngine::ready(char const* op) const {
  if (!stream_ || stream_->empty() || stream_->native() != native_stream_ ||
      stream_->device() != device_ || workspace_.empty())
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "stream is closed"));
  return {};
}

Fp8Input PrefillEngine::fp8_operand(unsigned m, unsigned k) const noexcept {
  // cuda/prefill.cu:502-508: codes [pm][k] at the front, scales after the
  // codes of the full capacity
  if (fp8_workspace_.empty() || !m || m > token_capacity_ || !k || k > kFp8MaxK || k % 128) return {};
  const std::uint64_t pm = (m + 127) / 128 * 128, cap = (token_capacity_ + 127) / 128 * 128;
  auto const* codes = static_cast<std::uint8_t const*>(fp8_workspace_.data());
  auto const* scales = reinterpret_cast<float const*>(codes + cap * kFp8MaxK);
  return {{codes, pm * k}, {scales, pm * (k / 128)}, unsigned(pm), k};
}

expected<void, Error> PrefillEngine::project_fp8(PrefillProjection const& d) {
  constexpr char const* op = "fp8.project";
  PrefillWeight const& w = d.weight;
  // cuda/prefill.cu:534-539: a residual exactly with the residual epilogue
  if ((d.epilogue == PrefillEpilogue::ResidualAddFp32) != (d.residual != nullptr) ||
      (d.epilogue != PrefillEpilogue::StoreBf16 && d.epilogue != PrefillEpilogue::StoreFp32 &&
       d.epilogue != PrefillEpilogue::ResidualAddFp32))
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.project",
                                 "input, output, position or epilogue contract mismatch"));
  if (w.quantizer != kDecodeQuantizerFp8V1 || w.n > 12288 || w.k > kFp8MaxK || w.n % 128 ||
      w.k % 256 || w.padded_n != w.n || w.padded_k != w.k ||
      w.codes_bytes != std::uint64_t(w.n) * w.k ||
      w.scales_bytes != std::uint64_t(w.n / 128) * (w.k / 128) * 4)
    return unexpected(make_error(ErrorCode::InvalidArgument, "prefill.weight",
                                 "weight, layout or token contract mismatch"));
  if (d.valid_tokens == 1) {  // cuda/prefill.cu:566-573: decode_mmv, no pack
    if (!d.packed.codes.empty() || !d.packed.scales.empty())
      return unexpected(make_error(ErrorCode::InvalidArgument, op, "unused decode pack"));
    const bool bf16 = d.epilogue == PrefillEpilogue::StoreBf16;
    DecodeMmvDesc desc;
    desc.layout = w.layout;
    desc.quantizer = w.quantizer;
    desc.n = desc.padded_n = w.n;
    desc.k = desc.padded_k = w.k;
    desc.epilogue = static_cast<DecodeEpilogue>(d.epilogue);
    desc.codes = decode_matrix_view(const_cast<void*>(w.codes), DecodeDtype::Fp8, w.layout, w.n, w.k,
                                    w.n, w.k, w.codes_bytes, 16);
    const auto units = static_cast<std::uint32_t>(w.scales_bytes / 4);
    desc.scales = decode_matrix_view(const_cast<void*>(w.scales), DecodeDtype::Fp32, w.layout, 1,
                                     units, 1, units, w.scales_bytes, 16);
    desc.input = decode_vector_view(const_cast<std::uint16_t*>(d.input), DecodeDtype::Bf16,
                                    kDecodeLayoutBf16VectorV0, w.k, std::uint64_t(w.k) * 2, 2, false);
    desc.output = decode_vector_view(d.output, bf16 ? DecodeDtype::Bf16 : DecodeDtype::Fp32,
                                     bf16 ? kDecodeLayoutBf16VectorV0 : kDecodeLayoutFp32VectorV0,
                                     w.n, std::uint64_t(w.n) * (bf16 ? 2 : 4), bf16 ? 2 : 4, true);
    if (d.residual)
      desc.residual = decode_vector_view(const_cast<float*>(d.residual), DecodeDtype::Fp32,
                                         kDecodeLayoutFp32VectorV0, w.n, std::uint64_t(w.n) * 4, 4,
                                         false);
    return fp8_decode(desc, *stream_);
  }
  // cuda/prefill.cu:574-578: the engine-owned operand, packed by the caller
  const Fp8Input owned = fp8_operand(d.valid_tokens, w.k);
  if (owned.codes.empty() || d.packed.codes.data() != owned.codes.data() ||
      d.packed.scales.data() != owned.scales.data() || d.packed.codes.size() != owned.codes.size() ||
      d.packed.scales.size() != owned.scales.size() || d.packed.m != owned.m || d.packed.k != owned.k)
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "plan-owned packed operand required"));
  const qw38_fp8_weight fw{static_cast<std::uint8_t const*>(w.codes), w.codes_bytes,
                           static_cast<float const*>(w.scales), w.scales_bytes / 4, w.n, w.k};
  const qw38_fp8_input fx = abi(owned);
  return from_abi(qw38_fp8_project(&fw, &fx, d.valid_tokens, d.output, d.residual,
                                   static_cast<int>(d.epilogue), native_stream_));
}

void* PrefillEngine::nvfp4_scratch() const noexcept {
  // qw38_prefill_mlp_workspace_bytes: the normalized and SwiGLU BF16 slabs,
  // then (256-byte aligned) the NVFP4 scratch of the token capacity
  const std::uint64_t slabs = (std::uint64_t(token_capacity_) * (5120u * 2u + 17408u * 2u) + 255u) / 256u * 256u;
  return static_cast<std::byte*>(const_cast<void*>(workspace_.data())) + slabs;
}

std::uint64_t PrefillEngine::nvfp4_scratch_bytes() const noexcept {
  return qw38_nvfp4_workspace_bytes(token_capacity_);
}

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
  if (d.weight.layout == kDecodeLayoutFp8V1) return project_fp8(d);
  const qw38_weight w = abi(d.weight);
  if (d.weight.layout == kDecodeLayoutNvFp4V1)  // cuda/prefill.cu:598-628: pack, W4A4, epilogue
    return from_abi(qw38_nvfp4_project(&w, d.input, d.valid_tokens, d.output, d.residual,
                                       static_cast<int>(d.epilogue), nvfp4_scratch(),
                                       nvfp4_scratch_bytes(), native_stream_));
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
  if (gate.layout == kDecodeLayoutNvFp4V1)  // cuda/prefill.cu:680-715: one pack, two W4A4 GEMMs
    return from_abi(qw38_nvfp4_paired_swiglu(&g, &u, normalized, swiglu, valid_tokens, nvfp4_scratch(),
                                             nvfp4_scratch_bytes(), native_stream_));
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
