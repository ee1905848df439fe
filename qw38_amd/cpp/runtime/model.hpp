// Device-resident weights of a `.qw38` artifact (interface subset of
// runtime/model.hpp in Enucatl/qw38: Model::upload, find_tensor, payload /
// scales views, device_bytes), plus this build's typed view of a quantized
// projection weight as a qw38::cuda::PrefillWeight.
//
// Upload policy (src/runtime/model.cpp:222-360 of the reference): every
// tensor span is validated on the host before any device allocation; spans
// shared by several records (aliases, identical offset/length) are uploaded
// once. Q4_K tiles in the reference layout 0x020D are uploaded byte for byte
// (the kernels consume 0x020D natively). Q4_K / Q6_K tensors stored as
// GGML-order super-blocks (this build's layouts 0x0250 / 0x0251) are repacked
// on the device at load time into the tiled layout the options name (0x020D
// or 0x0240 for Q4_K, 0x0241 for Q6_K); the repack changes only the byte
// order.
#pragma once

#include <cstdint>
#include <string_view>
#include <vector>

#include "cuda/buffer.hpp"
#include "cuda/prefill.hpp"
#include "cuda/stream.hpp"
#include "cuda/upload.hpp"
#include "format/artifact.hpp"
#include "qw38_hip.h"

namespace qw38::runtime {

using cuda::Error;
using cuda::expected;

struct ConstTensorView {
  void const* pointer{};
  std::uint64_t bytes{};
};

// Target of GGML-order Q4_K blocks. 0x020D by default: the decode kernels
// for M = 2..8 (int8 MFMA) and the fused M = 1 gate+up launch run on it, and
// the prefill MMQ runs within a few percent of 0x0240 there.
struct UploadOptions {
  std::uint16_t q4k_layout{QW38_LAYOUT_Q4K_CANDIDATE_V2};
};

class Model {
 public:
  Model(Model&&) noexcept = default;
  Model& operator=(Model&&) noexcept = default;
  ~Model() = default;
  Model(Model const&) = delete;
  Model& operator=(Model const&) = delete;

  [[nodiscard]] static expected<Model, Error> upload(qw38::format::Artifact const& artifact,
                                                     cuda::Stream const& stream,
                                                     UploadOptions options = {});

  [[nodiscard]] std::span<qw38::format::TensorRecord const> tensors() const noexcept {
    return records_;
  }
  [[nodiscard]] qw38::format::TensorRecord const* find_tensor(std::string_view name) const noexcept;
  [[nodiscard]] expected<ConstTensorView, Error> payload(std::string_view name) const;
  [[nodiscard]] expected<ConstTensorView, Error> scales(std::string_view name) const;
  // Q4_K (0x020D as stored, or repacked) and Q6_K (repacked to 0x0241)
  // projection weights, shaped [n out][k in].
  [[nodiscard]] expected<cuda::PrefillWeight, Error> weight(std::string_view name) const;

  [[nodiscard]] std::uint64_t device_bytes() const noexcept { return device_bytes_; }
  [[nodiscard]] int device() const noexcept { return device_; }

 private:
  Model() = default;
  struct Uploaded {
    std::uint32_t tensor_id{};
    ConstTensorView payload{};
    ConstTensorView scales{};
    bool tiled{};  // payload/scales are a tiled Q4_K / Q6_K weight
    cuda::PrefillWeight weight{};
  };
  std::vector<qw38::format::TensorRecord> records_;
  std::vector<cuda::DeviceBuffer> buffers_;
  std::vector<cuda::TiledWeight> tiled_;
  std::vector<Uploaded> uploaded_;
  std::uint64_t device_bytes_{0};
  int device_{-1};
};

}  // namespace qw38::runtime
