// Model::upload of a `.qw38` artifact (src/runtime/model.cpp:222-360 of
// Enucatl/qw38 defines the policy: host-side span checks before any device
// allocation, one upload per distinct span, aliases resolved to their owner).
#include "runtime/model.hpp"

#include <unordered_map>

#include "cuda/error.hpp"

namespace qw38::runtime {
namespace {

using qw38::format::TensorRecord;

Error malformed(std::string_view detail) {
  return cuda::make_error(cuda::ErrorCode::InvalidArgument, "model.upload", detail);
}

struct Geometry {
  std::uint32_t n{}, k{};
};

// [n][k] logical shape of a projection weight record.
expected<Geometry, Error> geometry(TensorRecord const& t) {
  if (t.shape.rank != 2 || t.shape.logical[0] == 0 || t.shape.logical[1] == 0 ||
      t.shape.logical[0] > (1u << 20) || t.shape.logical[1] > 65536)
    return cuda::unexpected(malformed("projection weight must be rank 2 [n][k]"));
  return Geometry{std::uint32_t(t.shape.logical[0]), std::uint32_t(t.shape.logical[1])};
}

}  // namespace

qw38::format::TensorRecord const* Model::find_tensor(std::string_view name) const noexcept {
  for (auto const& t : records_)
    if (t.logical_name == name) return &t;
  return nullptr;
}

expected<Model, Error> Model::upload(qw38::format::Artifact const& artifact, cuda::Stream const& stream,
                                     UploadOptions options) {
  namespace F = qw38::format;
  Model model;
  model.device_ = stream.device();
  model.records_.assign(artifact.tensors().begin(), artifact.tensors().end());
  if (options.q4k_layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 && options.q4k_layout != QW38_LAYOUT_Q4K_WAVE64)
    return cuda::unexpected(malformed("Q4_K target layout must be 0x020D or 0x0240"));

  // Host-side checks of every owner span before any device allocation.
  for (auto const& t : model.records_) {
    F::TensorRecord const* o = artifact.owner_of(t.tensor_id);
    if (!o) return cuda::unexpected(malformed("shared binding owner missing"));
    if (o != &t && o->tensor_id != t.tensor_id) continue;
    const bool blocks = t.layout == F::kLayoutQ4KGgmlBlocks || t.layout == F::kLayoutQ6KGgmlBlocks;
    if (blocks || t.layout == F::kLayoutQ4KTiles) {
      auto g = geometry(t);
      if (!g) return cuda::unexpected(g.error());
      const std::uint32_t pk = (g->k + 255) / 256 * 256, pn = (g->n + 7) / 8 * 8;
      if (blocks) {
        const bool q6 = t.layout == F::kLayoutQ6KGgmlBlocks;
        if (t.quantizer != (q6 ? F::kQuantizerQ6K : F::kQuantizerQ4K) || g->k % 256 || !t.scales.empty() ||
            t.payload.length != std::uint64_t(g->n) * (g->k / 256) * (q6 ? 210 : 144))
          return cuda::unexpected(malformed("GGML block tensor: quantizer, k % 256 or byte count mismatch"));
      } else if (t.quantizer != F::kQuantizerQ4K ||
                 t.payload.length != qw38_code_bytes(QW38_LAYOUT_Q4K_CANDIDATE_V2, pn, pk) ||
                 t.scales.length != qw38_scale_bytes(QW38_LAYOUT_Q4K_CANDIDATE_V2, pn, pk)) {
        return cuda::unexpected(malformed("0x020D tensor: quantizer or span sizes do not match its shape"));
      }
    }
    if (!t.payload.empty() && !artifact.span(t.logical_name, F::SpanKind::Payload))
      return cuda::unexpected(malformed("payload span unavailable"));
  }

  struct Key {
    std::uint64_t off, len;
    bool operator==(Key const&) const = default;
  };
  struct KeyHash {
    std::size_t operator()(Key const& k) const noexcept { return std::size_t(k.off ^ (k.len << 1)); }
  };
  std::unordered_map<Key, std::size_t, KeyHash> by_span;
  auto upload_span = [&](F::TensorRecord const& owner, F::SpanKind kind) -> expected<ConstTensorView, Error> {
    const F::ByteSpan s = kind == F::SpanKind::Payload ? owner.payload : owner.scales;
    if (s.empty()) return ConstTensorView{};
    const Key key{s.offset, s.length};
    if (auto it = by_span.find(key); it != by_span.end())
      return ConstTensorView{model.buffers_[it->second].data(), s.length};
    auto host = artifact.span(owner.logical_name, kind);
    if (!host) return cuda::unexpected(malformed(F::error_message(host.error())));
    auto buf = cuda::upload(*host, stream);
    if (!buf) return cuda::unexpected(buf.error());
    by_span.emplace(key, model.buffers_.size());
    model.device_bytes_ += buf->bytes();
    model.buffers_.push_back(std::move(*buf));
    return ConstTensorView{model.buffers_.back().data(), s.length};
  };

  std::unordered_map<std::uint32_t, std::size_t> tiled_of_owner;
  for (auto const& t : model.records_) {
    F::TensorRecord const* o = artifact.owner_of(t.tensor_id);
    Uploaded u;
    u.tensor_id = t.tensor_id;
    const bool blocks = o->layout == F::kLayoutQ4KGgmlBlocks || o->layout == F::kLayoutQ6KGgmlBlocks;
    if (blocks) {  // typed load-time repack, once per owner
      auto it = tiled_of_owner.find(o->tensor_id);
      if (it == tiled_of_owner.end()) {
        auto host = artifact.span(o->logical_name, F::SpanKind::Payload);
        if (!host) return cuda::unexpected(malformed(F::error_message(host.error())));
        const auto g = *geometry(*o);
        auto w = o->layout == F::kLayoutQ6KGgmlBlocks
                     ? cuda::upload_q6k_blocks(*host, g.n, g.k, stream)
                     : cuda::upload_q4k_blocks(*host, g.n, g.k, options.q4k_layout, stream);
        if (!w) return cuda::unexpected(w.error());
        model.device_bytes_ += w->codes.bytes() + w->scales.bytes();
        it = tiled_of_owner.emplace(o->tensor_id, model.tiled_.size()).first;
        model.tiled_.push_back(std::move(*w));
      }
      auto const& tw = model.tiled_[it->second];
      u.tiled = true;
      u.weight = tw.weight();
      u.payload = ConstTensorView{tw.codes.data(), tw.codes.bytes()};
      u.scales = ConstTensorView{tw.scales.data(), tw.scales.bytes()};
    } else {
      auto p = upload_span(*o, F::SpanKind::Payload);
      if (!p) return cuda::unexpected(p.error());
      auto s = upload_span(*o, F::SpanKind::Scales);
      if (!s) return cuda::unexpected(s.error());
      u.payload = *p;
      u.scales = *s;
      if (o->layout == F::kLayoutQ4KTiles) {
        const auto g = *geometry(*o);
        u.tiled = true;
        u.weight = cuda::PrefillWeight{p->pointer, s->pointer, QW38_LAYOUT_Q4K_CANDIDATE_V2, QW38_QUANTIZER_Q4K,
                                       g.n, g.k, (g.n + 7) / 8 * 8, (g.k + 255) / 256 * 256, p->bytes, s->bytes};
      }
    }
    model.uploaded_.push_back(u);
  }
  if (auto st = stream.sync(); !st) return cuda::unexpected(st.error());
  return model;
}

expected<ConstTensorView, Error> Model::payload(std::string_view name) const {
  auto const* t = find_tensor(name);
  if (!t) return cuda::unexpected(malformed("tensor not found"));
  for (auto const& u : uploaded_)
    if (u.tensor_id == t->tensor_id) return u.payload;
  return cuda::unexpected(malformed("uploaded tensor missing"));
}

expected<ConstTensorView, Error> Model::scales(std::string_view name) const {
  auto const* t = find_tensor(name);
  if (!t) return cuda::unexpected(malformed("tensor not found"));
  for (auto const& u : uploaded_)
    if (u.tensor_id == t->tensor_id) {
      if (!u.scales.pointer) return cuda::unexpected(malformed("tensor has no scales"));
      return u.scales;
    }
  return cuda::unexpected(malformed("uploaded tensor missing"));
}

expected<cuda::PrefillWeight, Error> Model::weight(std::string_view name) const {
  auto const* t = find_tensor(name);
  if (!t) return cuda::unexpected(malformed("tensor not found"));
  for (auto const& u : uploaded_)
    if (u.tensor_id == t->tensor_id) {
      if (!u.tiled) return cuda::unexpected(malformed("tensor is not a Q4_K / Q6_K projection weight"));
      return u.weight;
    }
  return cuda::unexpected(malformed("uploaded tensor missing"));
}

}  // namespace qw38::runtime
