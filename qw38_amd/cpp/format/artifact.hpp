// Minimal reader of the `.qw38` artifact container (interface subset of
// format/reader.hpp, format/schema.hpp and format/error.hpp in Enucatl/qw38):
// the 64-byte header, the manifest's prefix through the tensor directory and
// the shared bindings, and the manifest SHA-256 record that closes the
// manifest. The runtime-plan sections in between (graph bindings, state and
// scratch allocations) are not decoded: the projection path needs only the
// tensors. Validation happens before any view is handed out: header fields,
// exact file length, manifest bounds and digest, tensor spans inside the file,
// 256-byte aligned, in directory order and non-overlapping.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <memory>
#include <span>
#include <string>
#include <string_view>
#include <vector>

#include "qw38/expected.hpp"

namespace qw38::format {

using qw38::cuda::expected;
using qw38::cuda::unexpected;

// Same numbering as the reference's FormatErrorCode (format/error.hpp:9-50).
enum class FormatErrorCode : std::uint16_t {
  Truncated = 1,
  LeftoverBytes = 3,
  BadMagic = 4,
  UnsupportedContainerVersion = 5,
  UnsupportedManifestVersion = 6,
  ReservedNonzero = 8,
  Overflow = 9,
  Misaligned = 10,
  InvalidShape = 11,
  InvalidSpan = 12,
  SharedBinding = 16,
  InvalidHeader = 22,
  NameTooLong = 23,
  DuplicateId = 24,
  IoFailure = 25,
  OverlappingSpan = 31,
  IntegrityDigestMismatch = 33,
  MissingIntegrity = 34,
  TensorNotFound = 35,
  ResourceLimitExceeded = 36,
};

struct FormatError {
  FormatErrorCode code{};
  std::uint64_t offset{};
  std::string field;
  std::string detail;
};
[[nodiscard]] std::string error_message(FormatError const& error);

// Wire constants (format/constants.hpp:13-36 of the reference).
inline constexpr std::array<std::uint8_t, 8> kMagic{'Q', 'W', '3', '8', 'F', 'M', 'T', '\0'};
inline constexpr std::uint16_t kContainerVersionV0 = 1;
inline constexpr std::uint16_t kManifestVersionV0 = 1;
inline constexpr std::uint16_t kHeaderSizeV0 = 64;
inline constexpr std::uint64_t kSpanAlignment = 256;
inline constexpr std::uint8_t kMaxRank = 8;
inline constexpr std::uint16_t kMaxNameBytes = 1024;
inline constexpr std::uint64_t kMaxManifestBytesV0 = 16 * 1024 * 1024;
inline constexpr std::uint32_t kMaxTensorRecordsV0 = 4096;
inline constexpr std::uint32_t kMaxSharedBindingsV0 = 4096;
inline constexpr std::uint32_t kIntegrityRecordBytes = 56;
inline constexpr std::uint16_t kIntegritySha256Manifest = 0x0801;

// Layout / quantizer wire IDs this reader hands to the projection path: the
// reference's Q4_K tile layout, and this build's GGML-order super-block
// storage that Model::upload repacks on the device (no reference counterpart).
inline constexpr std::uint16_t kQuantizerQ4K = 0x0105;         // Q4KCandidateV2
inline constexpr std::uint16_t kQuantizerQ6K = 0x0140;         // this build
inline constexpr std::uint16_t kLayoutQ4KTiles = 0x020D;       // CudaQ4KCandidateV2
inline constexpr std::uint16_t kLayoutQ4KGgmlBlocks = 0x0250;  // this build: 144-byte blocks
inline constexpr std::uint16_t kLayoutQ6KGgmlBlocks = 0x0251;  // this build: 210-byte blocks

struct ByteSpan {
  std::uint64_t offset{};
  std::uint64_t length{};
  [[nodiscard]] bool empty() const noexcept { return length == 0; }
};

struct TensorShape {
  std::uint8_t rank{};
  std::array<std::uint64_t, kMaxRank> logical{};
  std::array<std::uint64_t, kMaxRank> padded{};
};

struct LogicalPhysicalMapping {
  std::uint16_t kind{};
  std::uint32_t tile_rows{};
  std::uint32_t tile_k{};
  std::uint32_t group_size{};
  std::uint32_t packed_bytes_per_tile_row{};
};

struct TensorRecord {
  std::uint32_t tensor_id{};
  std::string logical_name;
  TensorShape shape{};
  std::uint16_t storage{};
  std::uint16_t quantizer{};
  std::uint16_t layout{};
  LogicalPhysicalMapping mapping{};
  ByteSpan payload{};
  ByteSpan scales{};
};

struct SharedBinding {
  std::uint32_t owner_tensor_id{};
  std::uint32_t alias_tensor_id{};
  std::uint16_t role{};
};

struct ContainerHeader {
  std::uint16_t container_version{};
  std::uint16_t manifest_version{};
  std::uint16_t header_bytes{};
  std::uint64_t manifest_offset{};
  std::uint64_t manifest_length{};
};

enum class SpanKind : std::uint8_t { Payload, Scales };

// FIPS 180-4 SHA-256.
[[nodiscard]] std::array<std::uint8_t, 32> sha256(std::span<std::byte const> bytes);

// Host-only validated artifact: views exist only after validation succeeded.
class Artifact {
 public:
  Artifact(Artifact&&) noexcept;
  Artifact& operator=(Artifact&&) noexcept;
  ~Artifact();
  Artifact(Artifact const&) = delete;
  Artifact& operator=(Artifact const&) = delete;

  [[nodiscard]] static expected<Artifact, FormatError> open(std::filesystem::path path);
  [[nodiscard]] static expected<Artifact, FormatError> parse(std::span<std::byte const> bytes);

  [[nodiscard]] ContainerHeader const& header() const noexcept;
  [[nodiscard]] std::string const& compiler_ident() const noexcept;
  [[nodiscard]] std::span<TensorRecord const> tensors() const noexcept;
  [[nodiscard]] std::span<SharedBinding const> shared_bindings() const noexcept;
  [[nodiscard]] std::array<std::uint8_t, 32> const& manifest_digest() const noexcept;

  [[nodiscard]] TensorRecord const* find_tensor(std::string_view logical_name) const noexcept;
  [[nodiscard]] TensorRecord const* find_tensor(std::uint32_t tensor_id) const noexcept;
  // The tensor whose bytes back `tensor_id` (itself, or the owner it aliases).
  [[nodiscard]] TensorRecord const* owner_of(std::uint32_t tensor_id) const noexcept;

  // Borrowed views, valid for the lifetime of this Artifact.
  [[nodiscard]] expected<std::span<std::byte const>, FormatError> payload(
      std::string_view logical_name) const;
  [[nodiscard]] expected<std::span<std::byte const>, FormatError> scales(
      std::string_view logical_name) const;
  [[nodiscard]] expected<std::span<std::byte const>, FormatError> span(
      std::string_view logical_name, SpanKind kind) const;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
  explicit Artifact(std::unique_ptr<Impl> impl) noexcept;
};

}  // namespace qw38::format
