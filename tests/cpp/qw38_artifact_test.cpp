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

namespace F = qw38::format;
using namespace qw38::cuda;

namespace {

int g_failures = 0;
void expect(bool ok, std::string const& what) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  std::fflush(stdout);
  if (!ok) ++g_failures;
}

// ---- deterministic integers ------------------------------------------------------
struct Lcg {
  std::uint64_t s;
  std::uint32_t next() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return std::uint32_t(s >> 33);
  }
  int range(int lo, int hi) { return lo + int(next() % std::uint32_t(hi - lo + 1)); }
};

// ---- container writer -------------------------------------------------------------
struct WTensor {
  std::uint32_t id;
  std::string name;
  std::uint64_t n, k;
  std::uint16_t storage, quantizer, layout;
  std::vector<std::uint8_t> payload, scales;  // empty: alias / no scales
};
struct WShared {
  std::uint32_t owner, alias;
};

struct Bytes {
  std::vector<std::uint8_t> b;
  void u8(std::uint8_t v) { b.push_back(v); }
  void u16(std::uint16_t v) { for (int i = 0; i < 2; ++i) b.push_back(std::uint8_t(v >> (8 * i))); }
  void u32(std::uint32_t v) { for (int i = 0; i < 4; ++i) b.push_back(std::uint8_t(v >> (8 * i))); }
  void u64(std::uint64_t v) { for (int i = 0; i < 8; ++i) b.push_back(std::uint8_t(v >> (8 * i))); }
  void zeros(std::size_t n) { b.insert(b.end(), n, 0); }
  void name(std::string const& s) { u16(std::uint16_t(s.size())); b.insert(b.end(), s.begin(), s.end()); }
  void pad_to(std::size_t a) { while (b.size() % a) b.push_back(0); }
};

// payload_length_override != 0 writes that length into the first tensor's
// payload span (the bytes written stay the real ones): a sealed manifest with a
// span the reader must reject.
std::vector<std::uint8_t> write_artifact(std::vector<WTensor> const& ts, std::vector<WShared> const& sh,
                                         std::uint64_t payload_length_override = 0) {
  Bytes f;
  f.zeros(64);  // header, filled last
  struct Spans { std::uint64_t po, pl, so, sl; };
  std::vector<Spans> spans;
  for (auto const& t : ts) {
    Spans s{0, 0, 0, 0};
    if (!t.payload.empty()) {
      f.pad_to(256);
      s.po = f.b.size();
      s.pl = t.payload.size();
      f.b.insert(f.b.end(), t.payload.begin(), t.payload.end());
    }
    if (!t.scales.empty()) {
      f.pad_to(256);
      s.so = f.b.size();
      s.sl = t.scales.size();
      f.b.insert(f.b.end(), t.scales.begin(), t.scales.end());
    }
    spans.push_back(s);
  }
  f.pad_to(256);
  const std::uint64_t moff = f.b.size();
  Bytes m;
  m.u16(1);                 // manifest version
  m.name("qw38-amd-test");  // compiler ident, version, reserved
  m.u32(0); m.u32(1); m.u32(0); m.zeros(4);
  m.zeros(96);              // source, config, tokenizer hashes
  m.u16(0x0401); m.u16(1); m.u16(0x0B01); m.u16(0x0A01);  // precision policy V0: 1 binding
  m.u16(0x0501);            // scope: primary language
  m.u32(std::uint32_t(ts.size()));
  for (std::size_t i = 0; i < ts.size(); ++i) {
    auto const& t = ts[i];
    m.u32(t.id);
    m.name(t.name);
    m.u8(2); m.zeros(7);
    m.u64(t.n); m.u64((t.n + 7) / 8 * 8);
    m.u64(t.k); m.u64((t.k + 255) / 256 * 256);
    m.u16(t.storage); m.u16(t.quantizer); m.u16(t.layout); m.zeros(2);
    m.u16(0x0702); m.zeros(2); m.u32(8); m.u32(256); m.u32(32); m.u32(144);
    m.u64(spans[i].po);
    m.u64(i == 0 && payload_length_override ? payload_length_override : spans[i].pl);
    m.u64(spans[i].so); m.u64(spans[i].sl);
  }
  m.u32(std::uint32_t(sh.size()));
  for (auto const& s : sh) { m.u32(s.owner); m.u32(s.alias); m.u16(0x0901); m.zeros(2); }
  m.u32(0);  // graph bindings
  m.u32(0);  // state allocations
  m.u32(0);  // scratch allocations
  m.u32(1);  // integrity records: the manifest digest
  const std::uint64_t mlen = m.b.size() + 56;
  m.u16(0x0801); m.zeros(2); m.u32(0); m.u64(moff); m.u64(mlen); m.zeros(32);
  const auto digest = F::sha256(std::as_bytes(std::span(m.b)));
  std::memcpy(m.b.data() + m.b.size() - 32, digest.data(), 32);
  f.b.insert(f.b.end(), m.b.begin(), m.b.end());
  const char magic[8] = {'Q', 'W', '3', '8', 'F', 'M', 'T', '\0'};
  std::memcpy(f.b.data(), magic, 8);
  Bytes h;
  h.u16(1); h.u16(1); h.u16(64); h.zeros(2); h.u64(moff); h.u64(mlen);
  std::memcpy(f.b.data() + 8, h.b.data(), h.b.size());
  return f.b;
}

expected<F::Artifact, F::FormatError> parse(std::vector<std::uint8_t> const& v) {
  return F::Artifact::parse(std::as_bytes(std::span(v)));
}

// ---- quantized test tensors -------------------------------------------------------
// Logical Q4_K: codes [n][k] 0..15, per (row, super-block) d = dmin = fp16 1.0
// and 6-bit scales / mins; Q6_K: q [n][k] 0..63, int8 sub-block scales, d = 1.
struct Q4 {
  std::uint32_t n, k;
  std::vector<std::uint8_t> c;             // [n][k]
  std::vector<std::uint8_t> s, mn;         // [n][k/32]
};
struct Q6 {
  std::uint32_t n, k;
  std::vector<std::uint8_t> q;             // [n][k]
  std::vector<std::int8_t> sc;             // [n][k/16]
};

Q4 make_q4(std::uint32_t n, std::uint32_t k, std::uint64_t seed) {
  Lcg g{seed};
  Q4 w{n, k, std::vector<std::uint8_t>(std::size_t(n) * k), std::vector<std::uint8_t>(n * k / 32),
       std::vector<std::uint8_t>(n * k / 32)};
  for (auto& v : w.c) v = std::uint8_t(g.range(0, 15));
  for (auto& v : w.s) v = std::uint8_t(g.range(0, 31));
  for (auto& v : w.mn) v = std::uint8_t(g.range(0, 31));
  return w;
}
Q6 make_q6(std::uint32_t n, std::uint32_t k, std::uint64_t seed) {
  Lcg g{seed};
  Q6 w{n, k, std::vector<std::uint8_t>(std::size_t(n) * k), std::vector<std::int8_t>(n * k / 16)};
  for (auto& v : w.q) v = std::uint8_t(g.range(0, 63));
  for (auto& v : w.sc) v = std::int8_t(g.range(-12, 12));
  return w;
}

// 16 metadata bytes of one super-block: fp16 d, dmin (1.0) and the 12-byte
// 6-bit scale/min packing (llama.cpp get_scale_min_k4 inverse).
void q4_meta(Q4 const& w, std::uint32_t r, std::uint32_t kb, std::uint8_t* m) {
  m[0] = 0x00; m[1] = 0x3C; m[2] = 0x00; m[3] = 0x3C;
  std::uint8_t* p = m + 4;
  std::memset(p, 0, 12);
  for (int g = 0; g < 8; ++g) {
    const std::uint8_t s = w.s[(std::size_t(r) * w.k) / 32 + kb * 8 + g];
    const std::uint8_t mn = w.mn[(std::size_t(r) * w.k) / 32 + kb * 8 + g];
    if (g < 4) {
      p[g] |= s;
      p[g + 4] |= mn;
    } else {
      p[g + 4] |= std::uint8_t((s & 15) | ((mn & 15) << 4));
      p[g - 4] |= std::uint8_t((s >> 4) << 6);
      p[g] |= std::uint8_t((mn >> 4) << 6);
    }
  }
}

// Reference layout 0x020D (src/format/pack.cpp:216-262): tile row
// ((row/8) kbs + kb) 8 + row%8, 128 code bytes (byte j = c[2j] | c[2j+1] << 4)
// and 16 metadata bytes per tile row.
void pack_020d(Q4 const& w, std::vector<std::uint8_t>& codes, std::vector<std::uint8_t>& meta) {
  const std::uint32_t kbs = w.k / 256, pn = (w.n + 7) / 8 * 8;
  codes.assign(std::size_t(pn) * kbs * 128, 0);
  meta.assign(std::size_t(pn) * kbs * 16, 0);
  for (std::uint32_t r = 0; r < w.n; ++r)
    for (std::uint32_t kb = 0; kb < kbs; ++kb) {
      const std::size_t tr = (std::size_t(r / 8) * kbs + kb) * 8 + r % 8;
      for (int j = 0; j < 128; ++j)
        codes[tr * 128 + j] = std::uint8_t(w.c[std::size_t(r) * w.k + kb * 256 + 2 * j] |
                                           (w.c[std::size_t(r) * w.k + kb * 256 + 2 * j + 1] << 4));
      q4_meta(w, r, kb, &meta[tr * 16]);
    }
}

// GGML block_q4_K (144 B): meta 16 B, then qs: byte 32j + l holds code
// 64j + l (low nibble) and 64j + 32 + l (high nibble).
std::vector<std::uint8_t> ggml_q4(Q4 const& w) {
  const std::uint32_t kbs = w.k / 256;
  std::vector<std::uint8_t> out(std::size_t(w.n) * kbs * 144);
  for (std::uint32_t r = 0; r < w.n; ++r)
    for (std::uint32_t kb = 0; kb < kbs; ++kb) {
      std::uint8_t* b = &out[(std::size_t(r) * kbs + kb) * 144];
      q4_meta(w, r, kb, b);
      const std::uint8_t* c = &w.c[std::size_t(r) * w.k + kb * 256];
      for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 32; ++l) b[16 + 32 * j + l] = std::uint8_t(c[64 * j + l] | (c[64 * j + 32 + l] << 4));
    }
  return out;
}

// GGML block_q6_K (210 B): ql[128], qh[64], scales[16], fp16 d.
std::vector<std::uint8_t> ggml_q6(Q6 const& w) {
  const std::uint32_t kbs = w.k / 256;
  std::vector<std::uint8_t> out(std::size_t(w.n) * kbs * 210, 0);
  for (std::uint32_t r = 0; r < w.n; ++r)
    for (std::uint32_t kb = 0; kb < kbs; ++kb) {
      std::uint8_t* y = &out[(std::size_t(r) * kbs + kb) * 210];
      const std::uint8_t* L = &w.q[std::size_t(r) * w.k + kb * 256];
      for (int half = 0; half < 2; ++half) {
        const std::uint8_t* Lh = L + 128 * half;
        std::uint8_t* ql = y + 64 * half;
        std::uint8_t* qh = y + 128 + 32 * half;
        for (int l = 0; l < 32; ++l) {
          ql[l] = std::uint8_t((Lh[l] & 15) | ((Lh[l + 64] & 15) << 4));
          ql[l + 32] = std::uint8_t((Lh[l + 32] & 15) | ((Lh[l + 96] & 15) << 4));
          qh[l] = std::uint8_t((Lh[l] >> 4) | ((Lh[l + 32] >> 4) << 2) | ((Lh[l + 64] >> 4) << 4) |
                               ((Lh[l + 96] >> 4) << 6));
        }
      }
      std::memcpy(y + 192, &w.sc[(std::size_t(r) * w.k) / 16 + kb * 16], 16);
      y[208] = 0x00;
      y[209] = 0x3C;
    }
  return out;
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
