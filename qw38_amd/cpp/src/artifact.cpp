// Minimal `.qw38` container reader (format/reader.cpp, format/schema.cpp and
// format/wire.cpp of Enucatl/qw38 define the container; this file reads the
// subset the projection path needs). All integers are little-endian.
//
// Header (64 bytes): magic "QW38FMT\0", u16 container version (1), u16
// manifest version (1), u16 header bytes (64), 2 zero bytes, u64 manifest
// offset, u64 manifest length, 32 zero bytes. The manifest is the last thing
// in the file and ends with the 56-byte manifest integrity record, whose
// digest (its last 32 bytes) is the SHA-256 of the whole manifest with those
// 32 bytes zeroed.
//
// Manifest prefix: u16 version; compiler (u16-length name, u32 major, minor,
// patch, 4 zero bytes); source, config and tokenizer hashes (32 bytes each);
// precision policy (u16 id, u16 count, count x (u16 domain, u16 dtype)); u16
// scope; u32 tensor count and tensor records (u32 id, name, shape: u8 rank,
// 7 zero bytes, rank x (u64 logical, u64 padded); u16 storage, quantizer,
// layout, 2 zero bytes; mapping: u16 kind, 2 zero bytes, u32 tile rows, tile
// k, group size, packed bytes per tile row; payload and scale spans as u64
// offset + length); u32 shared-binding count and records (u32 owner, u32
// alias, u16 role, 2 zero bytes).
#include "format/artifact.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <limits>
#include <variant>

namespace qw38::format {
namespace {

FormatError err(FormatErrorCode code, std::uint64_t offset, std::string_view field,
                std::string_view detail) {
  return FormatError{code, offset, std::string(field), std::string(detail)};
}

// Bounds-checked little-endian cursor over the manifest.
class Cursor {
 public:
  Cursor(std::span<std::byte const> in, std::uint64_t base) : in_(in), base_(base) {}
  [[nodiscard]] std::uint64_t offset() const { return base_ + pos_; }

  template <class T>
  expected<T, FormatError> get(std::string_view field) {
    if (in_.size() - pos_ < sizeof(T))
      return unexpected(err(FormatErrorCode::Truncated, offset(), field, "manifest ends early"));
    T v = 0;
    for (std::size_t i = 0; i < sizeof(T); ++i)
      v |= T(std::to_integer<std::uint8_t>(in_[pos_ + i])) << (8 * i);
    pos_ += sizeof(T);
    return v;
  }
  expected<void, FormatError> zeros(std::size_t n, std::string_view field) {
    if (in_.size() - pos_ < n)
      return unexpected(err(FormatErrorCode::Truncated, offset(), field, "manifest ends early"));
    for (std::size_t i = 0; i < n; ++i)
      if (in_[pos_ + i] != std::byte{0})
        return unexpected(err(FormatErrorCode::ReservedNonzero, offset() + i, field,
                              "reserved bytes must be zero"));
    pos_ += n;
    return {};
  }
  expected<void, FormatError> skip(std::size_t n, std::string_view field) {
    if (in_.size() - pos_ < n)
      return unexpected(err(FormatErrorCode::Truncated, offset(), field, "manifest ends early"));
    pos_ += n;
    return {};
  }
  expected<std::string, FormatError> name(std::string_view field) {
    auto len = get<std::uint16_t>(field);
    if (!len) return unexpected(len.error());
    if (*len > kMaxNameBytes)
      return unexpected(err(FormatErrorCode::NameTooLong, offset() - 2, field,
                            "logical name exceeds 1024 bytes"));
    if (in_.size() - pos_ < *len)
      return unexpected(err(FormatErrorCode::Truncated, offset(), field, "manifest ends early"));
    std::string s(*len, '\0');
    std::memcpy(s.data(), in_.data() + pos_, *len);
    pos_ += *len;
    return s;
  }

 private:
  std::span<std::byte const> in_;
  std::uint64_t base_;
  std::size_t pos_ = 0;
};

#define QW38_TRY(var, expr)                          \
  auto var = (expr);                                 \
  if (!var) return unexpected(var.error())
#define QW38_TRY_VOID(expr)                          \
  do {                                               \
    auto qw38_st_ = (expr);                          \
    if (!qw38_st_) return unexpected(qw38_st_.error()); \
  } while (0)

expected<TensorRecord, FormatError> read_tensor(Cursor& c) {
  TensorRecord t;
  QW38_TRY(id, c.get<std::uint32_t>("tensor.id"));
  QW38_TRY(nm, c.name("tensor.logical_name"));
  QW38_TRY(rank, c.get<std::uint8_t>("tensor.shape"));
  QW38_TRY_VOID(c.zeros(7, "tensor.shape"));
  if (*rank == 0 || *rank > kMaxRank)
    return unexpected(err(FormatErrorCode::InvalidShape, c.offset(), "tensor.shape",
                          "rank must be 1..8"));
  t.tensor_id = *id;
  t.logical_name = std::move(*nm);
  t.shape.rank = *rank;
  for (int i = 0; i < *rank; ++i) {
    QW38_TRY(lg, c.get<std::uint64_t>("tensor.shape"));
    QW38_TRY(pd, c.get<std::uint64_t>("tensor.shape"));
    if (*lg == 0 || *pd < *lg)
      return unexpected(err(FormatErrorCode::InvalidShape, c.offset(), "tensor.shape",
                            "dimensions must be nonzero and padded >= logical"));
    t.shape.logical[i] = *lg;
    t.shape.padded[i] = *pd;
  }
  QW38_TRY(storage, c.get<std::uint16_t>("tensor.storage"));
  QW38_TRY(quant, c.get<std::uint16_t>("tensor.quantizer"));
  QW38_TRY(layout, c.get<std::uint16_t>("tensor.layout"));
  QW38_TRY_VOID(c.zeros(2, "tensor.reserved"));
  QW38_TRY(mk, c.get<std::uint16_t>("mapping.kind"));
  QW38_TRY_VOID(c.zeros(2, "mapping.reserved"));
  QW38_TRY(tr, c.get<std::uint32_t>("mapping.tile_rows"));
  QW38_TRY(tk, c.get<std::uint32_t>("mapping.tile_k"));
  QW38_TRY(gs, c.get<std::uint32_t>("mapping.group_size"));
  QW38_TRY(pb, c.get<std::uint32_t>("mapping.packed_bytes_per_tile_row"));
  QW38_TRY(po, c.get<std::uint64_t>("tensor.payload.offset"));
  QW38_TRY(pl, c.get<std::uint64_t>("tensor.payload.length"));
  QW38_TRY(so, c.get<std::uint64_t>("tensor.scales.offset"));
  QW38_TRY(sl, c.get<std::uint64_t>("tensor.scales.length"));
  t.storage = *storage;
  t.quantizer = *quant;
  t.layout = *layout;
  t.mapping = LogicalPhysicalMapping{*mk, *tr, *tk, *gs, *pb};
  t.payload = ByteSpan{*po, *pl};
  t.scales = ByteSpan{*so, *sl};
  return t;
}

// Span inside [lo, file_size), 256-byte aligned; empty spans use offset 0.
expected<void, FormatError> check_span(ByteSpan s, std::uint64_t file_size, std::string_view field) {
  if (s.empty()) {
    if (s.offset != 0)
      return unexpected(err(FormatErrorCode::InvalidSpan, s.offset, field,
                            "empty span must use offset 0"));
    return {};
  }
  if (s.offset % kSpanAlignment)
    return unexpected(err(FormatErrorCode::Misaligned, s.offset, field,
                          "span offset must be 256-byte aligned"));
  if (s.length > std::numeric_limits<std::uint64_t>::max() - s.offset)
    return unexpected(err(FormatErrorCode::Overflow, s.offset, field, "span end overflows"));
  if (s.offset + s.length > file_size)
    return unexpected(err(FormatErrorCode::InvalidSpan, s.offset, field, "span exceeds the file"));
  return {};
}

class Mapped {
 public:
  Mapped() = default;
  Mapped(Mapped&& o) noexcept : addr_(o.addr_), size_(o.size_) { o.addr_ = MAP_FAILED; o.size_ = 0; }
  Mapped& operator=(Mapped&& o) noexcept {
    if (this != &o) { reset(); addr_ = o.addr_; size_ = o.size_; o.addr_ = MAP_FAILED; o.size_ = 0; }
    return *this;
  }
  ~Mapped() { reset(); }
  static expected<Mapped, FormatError> open(std::filesystem::path const& path) {
    int fd = -1;
    do { fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC); } while (fd < 0 && errno == EINTR);
    if (fd < 0) return unexpected(err(FormatErrorCode::IoFailure, 0, "path", std::strerror(errno)));
    struct stat st {};
    if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode) || st.st_size < 0) {
      ::close(fd);
      return unexpected(err(FormatErrorCode::IoFailure, 0, "path", "artifact is not a regular file"));
    }
    Mapped m;
    m.size_ = std::size_t(st.st_size);
    if (m.size_ < kHeaderSizeV0) {
      ::close(fd);
      return unexpected(err(FormatErrorCode::Truncated, 0, "header",
                            "file is smaller than the 64-byte header"));
    }
    m.addr_ = ::mmap(nullptr, m.size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m.addr_ == MAP_FAILED) return unexpected(err(FormatErrorCode::IoFailure, 0, "path", std::strerror(errno)));
    return m;
  }
  [[nodiscard]] std::span<std::byte const> bytes() const {
    return addr_ == MAP_FAILED ? std::span<std::byte const>{}
                               : std::span<std::byte const>{static_cast<std::byte const*>(addr_), size_};
  }

 private:
  void reset() {
    if (addr_ != MAP_FAILED) ::munmap(addr_, size_);
    addr_ = MAP_FAILED;
    size_ = 0;
  }
  void* addr_ = MAP_FAILED;
  std::size_t size_ = 0;
};

struct Parsed {
  ContainerHeader header{};
  std::string compiler;
  std::vector<TensorRecord> tensors;
  std::vector<SharedBinding> shared;
  std::array<std::uint8_t, 32> digest{};
};

expected<void, FormatError> decode(std::span<std::byte const> bytes, Parsed& out);

}  // namespace

std::string error_message(FormatError const& e) {
  return "format error " + std::to_string(int(e.code)) + " at offset " + std::to_string(e.offset) + " (" +
         e.field + "): " + e.detail;
}

struct Artifact::Impl : Parsed {
  std::variant<Mapped, std::vector<std::byte>> storage;
  [[nodiscard]] std::span<std::byte const> bytes() const {
    if (auto const* m = std::get_if<Mapped>(&storage)) return m->bytes();
    return std::get<std::vector<std::byte>>(storage);
  }
};

Artifact::Artifact(std::unique_ptr<Impl> impl) noexcept : impl_(std::move(impl)) {}
Artifact::Artifact(Artifact&&) noexcept = default;
Artifact& Artifact::operator=(Artifact&&) noexcept = default;
Artifact::~Artifact() = default;

expected<Artifact, FormatError> Artifact::open(std::filesystem::path path) {
  auto m = Mapped::open(path);
  if (!m) return unexpected(m.error());
  auto impl = std::make_unique<Impl>();
  impl->storage = std::move(*m);
  if (auto st = decode(impl->bytes(), *impl); !st) return unexpected(st.error());
  return Artifact(std::move(impl));
}

expected<Artifact, FormatError> Artifact::parse(std::span<std::byte const> bytes) {
  auto impl = std::make_unique<Impl>();
  impl->storage = std::vector<std::byte>(bytes.begin(), bytes.end());
  if (auto st = decode(impl->bytes(), *impl); !st) return unexpected(st.error());
  return Artifact(std::move(impl));
}

namespace {

expected<void, FormatError> decode(std::span<std::byte const> bytes, Parsed& out) {
  if (bytes.size() < kHeaderSizeV0)
    return unexpected(err(FormatErrorCode::Truncated, 0, "header", "file is smaller than the 64-byte header"));
  // ---- header ----
  Cursor h(bytes.first(kHeaderSizeV0), 0);
  for (std::size_t i = 0; i < kMagic.size(); ++i)
    if (std::to_integer<std::uint8_t>(bytes[i]) != kMagic[i])
      return unexpected(err(FormatErrorCode::BadMagic, 0, "header.magic", "magic is not QW38FMT"));
  QW38_TRY_VOID(h.skip(8, "header.magic"));
  QW38_TRY(cv, h.get<std::uint16_t>("header.container_version"));
  QW38_TRY(mv, h.get<std::uint16_t>("header.manifest_version"));
  QW38_TRY(hb, h.get<std::uint16_t>("header.header_bytes"));
  QW38_TRY_VOID(h.zeros(2, "header.reserved0"));
  QW38_TRY(moff, h.get<std::uint64_t>("header.manifest_offset"));
  QW38_TRY(mlen, h.get<std::uint64_t>("header.manifest_length"));
  QW38_TRY_VOID(h.zeros(32, "header.reserved"));
  if (*cv != kContainerVersionV0)
    return unexpected(err(FormatErrorCode::UnsupportedContainerVersion, 8, "header.container_version",
                          "only container version 1 is supported"));
  if (*mv != kManifestVersionV0)
    return unexpected(err(FormatErrorCode::UnsupportedManifestVersion, 10, "header.manifest_version",
                          "only manifest version 1 is supported"));
  if (*hb != kHeaderSizeV0)
    return unexpected(err(FormatErrorCode::InvalidHeader, 12, "header.header_bytes", "header must be 64 bytes"));
  if (*moff < kHeaderSizeV0)
    return unexpected(err(FormatErrorCode::OverlappingSpan, *moff, "manifest", "manifest overlaps the header"));
  if (*mlen > kMaxManifestBytesV0)
    return unexpected(err(FormatErrorCode::ResourceLimitExceeded, *moff, "manifest",
                          "manifest exceeds the V0 size limit"));
  if (*mlen > std::numeric_limits<std::uint64_t>::max() - *moff)
    return unexpected(err(FormatErrorCode::Overflow, *moff, "manifest", "manifest end overflows"));
  const std::uint64_t mend = *moff + *mlen;
  if (mend > bytes.size())
    return unexpected(err(FormatErrorCode::Truncated, *moff, "manifest",
                          "file is shorter than the declared manifest"));
  if (mend < bytes.size())
    return unexpected(err(FormatErrorCode::LeftoverBytes, mend, "file",
                          "trailing bytes after the declared artifact"));
  out.header = ContainerHeader{*cv, *mv, *hb, *moff, *mlen};
  auto manifest = bytes.subspan(std::size_t(*moff), std::size_t(*mlen));

  // ---- manifest integrity: the final record covers the complete manifest ----
  if (*mlen < kIntegrityRecordBytes)
    return unexpected(err(FormatErrorCode::InvalidSpan, *moff, "manifest",
                          "manifest is smaller than one integrity record"));
  {
    Cursor r(manifest.last(kIntegrityRecordBytes), mend - kIntegrityRecordBytes);
    QW38_TRY(kind, r.get<std::uint16_t>("integrity.kind"));
    QW38_TRY_VOID(r.zeros(2, "integrity.reserved"));
    QW38_TRY(tid, r.get<std::uint32_t>("integrity.tensor"));
    QW38_TRY(ro, r.get<std::uint64_t>("integrity.offset"));
    QW38_TRY(rl, r.get<std::uint64_t>("integrity.length"));
    (void)tid;
    if (*kind != kIntegritySha256Manifest)
      return unexpected(err(FormatErrorCode::MissingIntegrity, *moff, "integrity",
                            "manifest SHA-256 record is required as the final record"));
    if (*ro != *moff || *rl != *mlen)
      return unexpected(err(FormatErrorCode::InvalidSpan, *ro, "integrity.region",
                            "manifest digest must cover the complete manifest"));
    std::vector<std::byte> canonical(manifest.begin(), manifest.end());
    std::fill(canonical.end() - 32, canonical.end(), std::byte{0});
    const auto actual = sha256(canonical);
    for (std::size_t i = 0; i < 32; ++i) out.digest[i] = std::to_integer<std::uint8_t>(manifest[*mlen - 32 + i]);
    if (actual != out.digest)
      return unexpected(err(FormatErrorCode::IntegrityDigestMismatch, *moff, "manifest",
                            "SHA-256 does not match the schema-declared region"));
  }

  // ---- manifest prefix through the tensor directory and shared bindings ----
  Cursor c(manifest, *moff);
  QW38_TRY(ver, c.get<std::uint16_t>("manifest.version"));
  if (*ver != kManifestVersionV0)
    return unexpected(err(FormatErrorCode::UnsupportedManifestVersion, *moff, "manifest.version",
                          "only manifest version 1 is supported"));
  QW38_TRY(ident, c.name("compiler.ident"));
  out.compiler = std::move(*ident);
  QW38_TRY_VOID(c.skip(12, "compiler.version"));
  QW38_TRY_VOID(c.zeros(4, "compiler.reserved"));
  QW38_TRY_VOID(c.skip(3 * 32, "hashes"));
  QW38_TRY(pid, c.get<std::uint16_t>("precision.id"));
  (void)pid;
  QW38_TRY(pcount, c.get<std::uint16_t>("precision.count"));
  QW38_TRY_VOID(c.skip(std::size_t(*pcount) * 4, "precision.bindings"));
  QW38_TRY(scope, c.get<std::uint16_t>("scope"));
  (void)scope;
  QW38_TRY(ntensors, c.get<std::uint32_t>("tensor_count"));
  if (*ntensors > kMaxTensorRecordsV0)
    return unexpected(err(FormatErrorCode::ResourceLimitExceeded, c.offset(), "tensor_count",
                          "too many tensor records"));
  out.tensors.reserve(*ntensors);
  for (std::uint32_t i = 0; i < *ntensors; ++i) {
    QW38_TRY(t, read_tensor(c));
    for (auto const& prev : out.tensors)
      if (prev.tensor_id == t->tensor_id || prev.logical_name == t->logical_name)
        return unexpected(err(FormatErrorCode::DuplicateId, c.offset(), "tensor.id",
                              "duplicate tensor id or logical name"));
    out.tensors.push_back(std::move(*t));
  }
  QW38_TRY(nshared, c.get<std::uint32_t>("shared_count"));
  if (*nshared > kMaxSharedBindingsV0)
    return unexpected(err(FormatErrorCode::ResourceLimitExceeded, c.offset(), "shared_count",
                          "too many shared bindings"));
  for (std::uint32_t i = 0; i < *nshared; ++i) {
    QW38_TRY(owner, c.get<std::uint32_t>("shared.owner"));
    QW38_TRY(alias, c.get<std::uint32_t>("shared.alias"));
    QW38_TRY(role, c.get<std::uint16_t>("shared.role"));
    QW38_TRY_VOID(c.zeros(2, "shared.reserved"));
    out.shared.push_back(SharedBinding{*owner, *alias, *role});
  }
  if (c.offset() > mend - kIntegrityRecordBytes)
    return unexpected(err(FormatErrorCode::InvalidSpan, c.offset(), "manifest",
                          "tensor directory overlaps the integrity record"));

  // ---- shared bindings resolve to owners with bytes; aliases carry none ----
  for (auto const& b : out.shared) {
    auto find = [&](std::uint32_t id) -> TensorRecord const* {
      for (auto const& t : out.tensors)
        if (t.tensor_id == id) return &t;
      return nullptr;
    };
    TensorRecord const* o = find(b.owner_tensor_id);
    TensorRecord const* a = find(b.alias_tensor_id);
    if (!o || !a || o == a || o->payload.empty() || !a->payload.empty() || !a->scales.empty())
      return unexpected(err(FormatErrorCode::SharedBinding, *moff, "shared",
                            "shared binding must alias a byte-less tensor to an owner with a payload"));
  }

  // ---- tensor spans: in the file, aligned, directory order, no overlap ----
  struct Occ { std::uint64_t off, len; };
  std::vector<Occ> occ{{0, kHeaderSizeV0}, {*moff, *mlen}};
  std::uint64_t prev_end = 0;
  for (auto const& t : out.tensors) {
    QW38_TRY_VOID(check_span(t.payload, bytes.size(), "tensor.payload"));
    QW38_TRY_VOID(check_span(t.scales, bytes.size(), "tensor.scales"));
    if (!t.payload.empty()) {
      if (t.payload.offset < prev_end)
        return unexpected(err(FormatErrorCode::InvalidSpan, t.payload.offset, "tensor.payload",
                              "owner payload spans must follow tensor directory order"));
      prev_end = t.payload.offset + t.payload.length;
      occ.push_back({t.payload.offset, t.payload.length});
    }
    if (!t.scales.empty()) {
      if (t.scales.offset < prev_end)
        return unexpected(err(FormatErrorCode::InvalidSpan, t.scales.offset, "tensor.scales",
                              "scale span must follow its tensor payload"));
      prev_end = t.scales.offset + t.scales.length;
      occ.push_back({t.scales.offset, t.scales.length});
    }
  }
  std::sort(occ.begin(), occ.end(), [](Occ a, Occ b) { return a.off < b.off; });
  for (std::size_t i = 1; i < occ.size(); ++i)
    if (occ[i].off < occ[i - 1].off + occ[i - 1].len)
      return unexpected(err(FormatErrorCode::OverlappingSpan, occ[i].off, "spans",
                            "header, payload, scale, or manifest spans overlap"));
  return {};
}

}  // namespace

ContainerHeader const& Artifact::header() const noexcept { return impl_->header; }
std::string const& Artifact::compiler_ident() const noexcept { return impl_->compiler; }
std::span<TensorRecord const> Artifact::tensors() const noexcept { return impl_->tensors; }
std::span<SharedBinding const> Artifact::shared_bindings() const noexcept { return impl_->shared; }
std::array<std::uint8_t, 32> const& Artifact::manifest_digest() const noexcept { return impl_->digest; }

TensorRecord const* Artifact::find_tensor(std::string_view name) const noexcept {
  for (auto const& t : impl_->tensors)
    if (t.logical_name == name) return &t;
  return nullptr;
}
TensorRecord const* Artifact::find_tensor(std::uint32_t id) const noexcept {
  for (auto const& t : impl_->tensors)
    if (t.tensor_id == id) return &t;
  return nullptr;
}
TensorRecord const* Artifact::owner_of(std::uint32_t id) const noexcept {
  for (auto const& b : impl_->shared)
    if (b.alias_tensor_id == id) return find_tensor(b.owner_tensor_id);
  return find_tensor(id);
}

expected<std::span<std::byte const>, FormatError> Artifact::span(std::string_view name, SpanKind kind) const {
  TensorRecord const* t = find_tensor(name);
  if (!t) return unexpected(err(FormatErrorCode::TensorNotFound, 0, "tensor", "tensor not found"));
  TensorRecord const* o = owner_of(t->tensor_id);
  const ByteSpan s = kind == SpanKind::Payload ? o->payload : o->scales;
  if (s.empty()) return std::span<std::byte const>{};
  return impl_->bytes().subspan(std::size_t(s.offset), std::size_t(s.length));
}
expected<std::span<std::byte const>, FormatError> Artifact::payload(std::string_view name) const {
  return span(name, SpanKind::Payload);
}
expected<std::span<std::byte const>, FormatError> Artifact::scales(std::string_view name) const {
  return span(name, SpanKind::Scales);
}

}  // namespace qw38::format
