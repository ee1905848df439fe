// `.qw38` reader and Model::upload test (the reference's
// tests/format_reader_test.cpp, format_reader_digest_test.cpp and
// format_sha256_test.cpp cover the same contract for its reader).
//
// A small container writer below builds artifacts in the wire format
// (header, 256-byte aligned tensor spans, manifest prefix, zero graph /
// state / scratch sections, and the closing manifest SHA-256 record). Host
// checks: SHA-256 known-answer vectors (FIPS 180-2 examples), round trip of
// every record field, alias resolution, and one typed rejection per broken
// invariant. GPU checks (without --host): Model::upload of a Q4_K 0x020D
// tensor (bytes on the device equal the file bytes), a GGML-order Q4_K
// tensor repacked to 0x0240 and a GGML-order Q6_K tensor repacked to 0x0241;
// q4k_q8_project on each uploaded weight with integer-valued activations
// (every Q8 group peaks at +-127, so a = 1) must equal the exact integer
// closed form computed here.
//
// Run: qw38_artifact_test [--host]; one line per check, nonzero exit on
// any failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "cuda/buffer.hpp"
#include "cuda/copy.hpp"
#include "cuda/q4k_q8.hpp"
#include "cuda/stream.hpp"
#include "format/artifact.hpp"
#include "runtime/model.hpp"
#include "artifact_fixture.hpp"

namespace F = qw38::format;
using namespace qw38::cuda;
using namespace fixture;

namespace {

int g_failures = 0;
void expect(bool ok, std::string const& what) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  std::fflush(stdout);
  if (!ok) ++g_failures;
}

// ---- host checks ------------------------------------------------------------------
std::string hex(std::array<std::uint8_t, 32> const& h) {
  static const char* d = "0123456789abcdef";
  std::string s;
  for (auto v : h) { s += d[v >> 4]; s += d[v & 15]; }
  return s;
}

void test_sha256() {
  auto h = [](std::string const& s) { return hex(F::sha256(std::as_bytes(std::span(s.data(), s.size())))); };
  expect(h("") == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855", "SHA-256 of empty message");
  expect(h("abc") == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad", "SHA-256 of abc");
  expect(h("abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq") ==
             "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
         "SHA-256 of the 448-bit FIPS example");
  expect(h(std::string(1000000, 'a')) == "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0",
         "SHA-256 of one million 'a'");
}

std::vector<WTensor> fixture_tensors() {
  const Q4 q4 = make_q4(40, 512, 11);
  std::vector<std::uint8_t> co, mo;
  pack_020d(q4, co, mo);
  return {
      {1, "layers.0.mlp.gate_proj.weight", 40, 512, 0x0001, F::kQuantizerQ4K, F::kLayoutQ4KTiles, co, mo},
      {2, "layers.0.mlp.up_proj.weight", 24, 768, 0x0001, F::kQuantizerQ4K, F::kLayoutQ4KGgmlBlocks,
       ggml_q4(make_q4(24, 768, 12)), {}},
      {3, "layers.0.mlp.down_proj.weight", 16, 1024, 0x0002, F::kQuantizerQ6K, F::kLayoutQ6KGgmlBlocks,
       ggml_q6(make_q6(16, 1024, 13)), {}},
      {4, "mtp.layers.0.mlp.gate_proj.weight", 40, 512, 0x0001, F::kQuantizerQ4K, F::kLayoutQ4KTiles, {}, {}},
  };
}

void test_reader() {
  const auto ts = fixture_tensors();
  const std::vector<WShared> sh{{1, 4}};
  const auto bytes = write_artifact(ts, sh);
  auto a = parse(bytes);
  expect(bool(a), "reader accepts a well-formed artifact" + (a ? std::string() : ": " + F::error_message(a.error())));
  if (!a) return;
  expect(a->tensors().size() == 4 && a->compiler_ident() == "qw38-amd-test", "tensor directory and compiler ident");
  bool fields = true;
  for (std::size_t i = 0; i < ts.size(); ++i) {
    auto const& r = a->tensors()[i];
    fields = fields && r.tensor_id == ts[i].id && r.logical_name == ts[i].name && r.shape.rank == 2 &&
             r.shape.logical[0] == ts[i].n && r.shape.logical[1] == ts[i].k && r.storage == ts[i].storage &&
             r.quantizer == ts[i].quantizer && r.layout == ts[i].layout && r.payload.length == ts[i].payload.size() &&
             r.scales.length == ts[i].scales.size() && r.payload.offset % 256 == 0;
  }
  expect(fields, "every record field round-trips");
  auto p = a->payload("layers.0.mlp.gate_proj.weight");
  expect(p && p->size() == ts[0].payload.size() && std::memcmp(p->data(), ts[0].payload.data(), p->size()) == 0,
         "payload view equals the written bytes");
  auto s = a->scales("layers.0.mlp.gate_proj.weight");
  expect(s && std::memcmp(s->data(), ts[0].scales.data(), s->size()) == 0, "scale view equals the written bytes");
  auto alias = a->payload("mtp.layers.0.mlp.gate_proj.weight");
  expect(alias && p && alias->data() == p->data(), "alias resolves to its owner's bytes");
  expect(!a->payload("missing.weight") && a->payload("missing.weight").error().code == F::FormatErrorCode::TensorNotFound,
         "unknown tensor is TensorNotFound");
  // the digest in the file equals an independent SHA-256 over the manifest
  // with its own 32 digest bytes zeroed
  const auto& hdr = a->header();
  std::vector<std::uint8_t> man(bytes.begin() + std::ptrdiff_t(hdr.manifest_offset), bytes.end());
  std::fill(man.end() - 32, man.end(), 0);
  expect(F::sha256(std::as_bytes(std::span(man))) == a->manifest_digest(), "manifest digest covers the manifest");

  auto rejects = [&](std::vector<std::uint8_t> v, F::FormatErrorCode code, std::string const& what) {
    auto r = parse(v);
    expect(!r && r.error().code == code,
           what + (r ? " (accepted)" : " (" + F::error_message(r.error()) + ")"));
  };
  auto v = bytes;
  v[0] = 'X';
  rejects(v, F::FormatErrorCode::BadMagic, "bad magic rejected");
  v = bytes;
  v[8] = 2;
  rejects(v, F::FormatErrorCode::UnsupportedContainerVersion, "container version 2 rejected");
  v = bytes;
  v.push_back(0);
  rejects(v, F::FormatErrorCode::LeftoverBytes, "trailing byte rejected");
  v = bytes;
  v.pop_back();
  rejects(v, F::FormatErrorCode::Truncated, "truncated manifest rejected");
  v = std::vector<std::uint8_t>(bytes.begin(), bytes.begin() + 40);
  rejects(v, F::FormatErrorCode::Truncated, "file shorter than the header rejected");
  v = bytes;
  v[hdr.manifest_offset + 3] ^= 1;  // inside the compiler ident
  rejects(v, F::FormatErrorCode::IntegrityDigestMismatch, "manifest bit flip rejected by the digest");
  v = bytes;
  v[40] = 1;  // header reserved byte
  rejects(v, F::FormatErrorCode::ReservedNonzero, "nonzero header reserved byte rejected");

  // broken spans, written with a valid digest so only the span checks fire
  auto ts2 = ts;
  ts2[1].payload.resize(ts2[1].payload.size() + 1);  // next span stays 256-aligned: no overlap
  {
    auto w = write_artifact(ts2, sh);
    auto r = parse(w);
    expect(bool(r), "odd-length payload still parses (length checks belong to the upload)");
  }
  {
    auto r = parse(write_artifact(ts, sh, 0, [](std::vector<WSpans>& sp) { sp[1].po += 16; }));
    expect(!r && r.error().code == F::FormatErrorCode::Misaligned, "span offset off the 256-byte grid rejected");
  }
  {
    // the second payload starts 256 bytes into the first
    auto r = parse(write_artifact(ts, sh, 0, [](std::vector<WSpans>& sp) { sp[1].po = sp[0].po + 256; }));
    expect(!r && (r.error().code == F::FormatErrorCode::OverlappingSpan ||
                  r.error().code == F::FormatErrorCode::InvalidSpan),
           "overlapping payload spans rejected" + (r ? std::string() : " (" + F::error_message(r.error()) + ")"));
  }
  {
    // alias record whose owner has no payload
    auto r = parse(write_artifact(ts, {{4, 1}}));
    expect(!r && r.error().code == F::FormatErrorCode::SharedBinding, "alias of a byte-less owner rejected");
  }
  {
    // duplicate logical name
    auto t3 = ts;
    t3[2].name = t3[1].name;
    auto r = parse(write_artifact(t3, sh));
    expect(!r && r.error().code == F::FormatErrorCode::DuplicateId, "duplicate logical name rejected");
  }
  {
    auto r = parse(write_artifact(ts, sh, std::uint64_t(1) << 40));
    expect(!r && r.error().code == F::FormatErrorCode::InvalidSpan,
           "payload span past the file rejected" + (r ? std::string(" (accepted)") : " (" + F::error_message(r.error()) + ")"));
  }
  {
    auto r = parse(write_artifact(ts, sh, ts[0].payload.size() + 300));
    expect(!r && r.error().code == F::FormatErrorCode::InvalidSpan,
           "payload span running into the scale span rejected" +
               (r ? std::string(" (accepted)") : " (" + F::error_message(r.error()) + ")"));
  }
}

// ---- GPU checks -------------------------------------------------------------------
// y[t][r] = sum_k W[r][k] x[t][k] exactly, for the integer weights above.
std::vector<double> exact_q4(Q4 const& w, std::vector<int> const& x, std::uint32_t m) {
  std::vector<double> y(std::size_t(m) * w.n, 0.0);
  for (std::uint32_t t = 0; t < m; ++t)
    for (std::uint32_t r = 0; r < w.n; ++r) {
      long acc = 0;
      for (std::uint32_t kk = 0; kk < w.k; ++kk) {
        const std::size_t gi = (std::size_t(r) * w.k + kk) / 32;
        acc += long(int(w.s[gi]) * int(w.c[std::size_t(r) * w.k + kk]) - int(w.mn[gi])) * x[std::size_t(t) * w.k + kk];
      }
      y[std::size_t(t) * w.n + r] = double(acc);
    }
  return y;
}
std::vector<double> exact_q6(Q6 const& w, std::vector<int> const& x, std::uint32_t m) {
  std::vector<double> y(std::size_t(m) * w.n, 0.0);
  for (std::uint32_t t = 0; t < m; ++t)
    for (std::uint32_t r = 0; r < w.n; ++r) {
      long acc = 0;
      for (std::uint32_t kk = 0; kk < w.k; ++kk)
        acc += long(w.sc[(std::size_t(r) * w.k + kk) / 16]) * (int(w.q[std::size_t(r) * w.k + kk]) - 32) *
               x[std::size_t(t) * w.k + kk];
      y[std::size_t(t) * w.n + r] = double(acc);
    }
  return y;
}

// Integer activations in {-1, 0, 1} with one +-127 per K32 group.
std::vector<int> int_rows(std::uint32_t m, std::uint32_t k, std::uint64_t seed) {
  Lcg g{seed};
  std::vector<int> x(std::size_t(m) * k);
  for (auto& v : x) v = g.range(-1, 1);
  for (std::uint32_t t = 0; t < m; ++t)
    for (std::uint32_t grp = 0; grp < k / 32; ++grp)
      x[std::size_t(t) * k + grp * 32 + g.range(0, 31)] = (g.next() & 1) ? 127 : -127;
  return x;
}

std::uint16_t bf16_of_int(int v) {  // exact for |v| <= 256
  const float f = float(v);
  std::uint32_t u;
  std::memcpy(&u, &f, 4);
  return std::uint16_t(u >> 16);
}

template <class T>
DeviceBuffer dev(std::vector<T> const& v, Stream const& s) {
  auto b = upload(std::as_bytes(std::span<T const>(v)), s);
  if (!b) { std::printf("FAIL upload: %s\n", error_message(b.error()).c_str()); std::exit(2); }
  return std::move(*b);
}

bool project_exact(PrefillWeight const& w, std::vector<int> const& x, std::uint32_t m,
                   std::vector<double> const& want, Stream const& s) {
  const std::uint32_t pk = w.padded_k, groups = pk / 32;
  std::vector<std::uint16_t> xb(x.size());
  for (std::size_t i = 0; i < x.size(); ++i) xb[i] = bf16_of_int(x[i]);
  auto dx = dev(xb, s);
  auto codes = DeviceBuffer::allocate(std::size_t(m) * pk);
  auto sc = DeviceBuffer::allocate(std::size_t(m) * groups * 4);
  auto su = DeviceBuffer::allocate(std::size_t(m) * groups * 4);
  auto flag = DeviceBuffer::allocate(4);
  auto out = DeviceBuffer::allocate(std::size_t(m) * w.n * 4);
  if (!codes || !sc || !su || !flag || !out) return false;
  Q8Input q{{static_cast<std::int8_t*>(codes->data()), std::size_t(m) * pk},
            {static_cast<float*>(sc->data()), std::size_t(m) * groups},
            {static_cast<std::int32_t*>(su->data()), std::size_t(m) * groups}, m, w.k, pk};
  if (!pack_q8({static_cast<std::uint16_t const*>(dx.data()), xb.size()}, q,
               {static_cast<int*>(flag->data()), 1}, s))
    return false;
  if (!q4k_q8_project(w, q, {static_cast<float*>(out->data()), std::size_t(m) * w.n}, s)) return false;
  std::vector<float> y(std::size_t(m) * w.n);
  if (!copy_d2h(y.data(), out->data(), y.size() * 4, s) || !s.sync()) return false;
  for (std::size_t i = 0; i < y.size(); ++i)
    if (double(y[i]) != want[i]) {
      std::printf("  mismatch at %zu: %.1f vs %.1f\n", i, double(y[i]), want[i]);
      return false;
    }
  return true;
}

void test_upload(Stream const& s) {
  const auto ts = fixture_tensors();
  const auto bytes = write_artifact(ts, {{1, 4}});
  auto a = parse(bytes);
  if (!a) { expect(false, "parse"); return; }
  for (std::uint16_t layout : {std::uint16_t(QW38_LAYOUT_Q4K_WAVE64), std::uint16_t(QW38_LAYOUT_Q4K_CANDIDATE_V2)}) {
    auto model = qw38::runtime::Model::upload(*a, s, {layout});
    expect(bool(model), "Model::upload" + (model ? std::string() : ": " + error_message(model.error())));
    if (!model) return;
    // 0x020D tensor: device bytes are the file bytes
    auto p = model->payload("layers.0.mlp.gate_proj.weight");
    std::vector<std::uint8_t> back(ts[0].payload.size());
    const bool copied = p && copy_d2h(back.data(), p->pointer, back.size(), s) && s.sync();
    expect(copied && back == ts[0].payload, "0x020D payload uploaded byte for byte");
    auto pa = model->payload("mtp.layers.0.mlp.gate_proj.weight");
    expect(pa && p && pa->pointer == p->pointer, "alias shares the owner's device buffer");
    const std::uint32_t m = 5;
    {
      auto w = model->weight("layers.0.mlp.gate_proj.weight");
      const Q4 q4 = make_q4(40, 512, 11);
      const auto x = int_rows(m, 512, 21);
      expect(w && w->layout == QW38_LAYOUT_Q4K_CANDIDATE_V2 && project_exact(*w, x, m, exact_q4(q4, x, m), s),
             "0x020D weight from the artifact: q4k_q8_project exact");
    }
    {
      auto w = model->weight("layers.0.mlp.up_proj.weight");
      const Q4 q4 = make_q4(24, 768, 12);
      const auto x = int_rows(m, 768, 22);
      expect(w && w->layout == layout && project_exact(*w, x, m, exact_q4(q4, x, m), s),
             "GGML Q4_K blocks repacked to " + std::to_string(layout) + " at load: project exact");
      const auto x1 = int_rows(1, 768, 23);
      expect(w && project_exact(*w, x1, 1, exact_q4(q4, x1, 1), s), "  ... and the M=1 GEMV exact");
    }
    {
      auto w = model->weight("layers.0.mlp.down_proj.weight");
      const Q6 q6 = make_q6(16, 1024, 13);
      for (std::uint32_t mm : {1u, 4u, 12u}) {
        const auto x = int_rows(mm, 1024, 24 + mm);
        expect(w && w->layout == QW38_LAYOUT_Q6K_WAVE64 && project_exact(*w, x, mm, exact_q6(q6, x, mm), s),
               "GGML Q6_K blocks repacked to 0x0241 at load: project exact, M=" + std::to_string(mm));
      }
    }
    expect(!model->weight("missing") && model->device_bytes() > 0, "unknown weight rejected, device bytes counted");
  }
  // an 0x020D tensor whose spans do not match its shape is rejected before upload
  auto bad = ts;
  bad[0].scales.resize(bad[0].scales.size() - 16);
  auto b2 = parse(write_artifact(bad, {{1, 4}}));
  auto model = b2 ? qw38::runtime::Model::upload(*b2, s) : expected<qw38::runtime::Model, Error>(unexpected(Error{}));
  expect(b2 && !model, "0x020D span sizes checked against the shape before any allocation");
}

}  // namespace

int main(int argc, char** argv) {
  const bool host_only = argc > 1 && std::strcmp(argv[1], "--host") == 0;
  std::printf("== sha256\n");
  test_sha256();
  std::printf("== reader\n");
  test_reader();
  if (!host_only) {
    auto stream = Stream::create();
    if (!stream) { std::printf("FAIL stream\n"); return 2; }
    std::printf("== upload\n");
    test_upload(*stream);
    if (!stream->sync()) return 2;
  }
  std::printf("%d failure(s)\n", g_failures);
  return g_failures == 0 ? 0 : 1;
}
