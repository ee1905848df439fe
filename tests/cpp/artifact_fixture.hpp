// Test fixtures shared by the C++ artifact and runtime tests: a writer of
// `.qw38` containers in the wire format (header, 256-byte aligned tensor
// spans, manifest prefix, zero graph / state / scratch sections and the
// closing manifest SHA-256 record) and deterministic Q4_K / Q6_K weights in
// the reference layout 0x020D and in GGML block order.
#pragma once

#include <cstdint>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "format/artifact.hpp"

namespace fixture {

namespace F = qw38::format;

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

// Payload / scale spans of one tensor record (offset, length).
struct WSpans {
  std::uint64_t po, pl, so, sl;
};

// payload_length_override != 0 writes that length into the first tensor's
// payload span (the bytes written stay the real ones); edit, when given,
// rewrites the recorded spans before the manifest is sealed: manifests with a
// valid digest and spans the reader must reject.
inline std::vector<std::uint8_t> write_artifact(std::vector<WTensor> const& ts, std::vector<WShared> const& sh,
                                         std::uint64_t payload_length_override = 0,
                                         std::function<void(std::vector<WSpans>&)> const& edit = {}) {
  Bytes f;
  f.zeros(64);  // header, filled last
  using Spans = WSpans;
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
  if (edit) edit(spans);
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

inline F::expected<F::Artifact, F::FormatError> parse(std::vector<std::uint8_t> const& v) {
  return F::Artifact::parse(std::as_bytes(std::span(v)));
}

// ---- quantized test tensors -------------------------------------------------------
// Logical Q4_K: codes [n][k] 0..15, per (row, super-block) d = dmin = fp16 1.0
// and 6-bit scales / mins; Q6_K: q [n][k] 0..63, int8 sub-block scales, d = 1.
struct Q4 {
  std::uint32_t n, k;
  std::vector<std::uint8_t> c;             // [n][k]
  std::vector<std::uint8_t> s, mn;         // [n][k/32]
  std::uint16_t d{0x3C00}, dmin{0x3C00};   // fp16 bits, every super-block
};
struct Q6 {
  std::uint32_t n, k;
  std::vector<std::uint8_t> q;             // [n][k]
  std::vector<std::int8_t> sc;             // [n][k/16]
  std::uint16_t d{0x3C00};                 // fp16 bits, every super-block
};

inline Q4 make_q4(std::uint32_t n, std::uint32_t k, std::uint64_t seed, int smax = 31,
           std::uint16_t d_bits = 0x3C00, std::uint16_t dmin_bits = 0x3C00) {
  Lcg g{seed};
  Q4 w{n, k, std::vector<std::uint8_t>(std::size_t(n) * k), std::vector<std::uint8_t>(std::size_t(n) * k / 32),
       std::vector<std::uint8_t>(std::size_t(n) * k / 32)};
  for (auto& v : w.c) v = std::uint8_t(g.range(0, 15));
  for (auto& v : w.s) v = std::uint8_t(g.range(0, smax));
  for (auto& v : w.mn) v = std::uint8_t(g.range(0, smax));
  w.d = d_bits;
  w.dmin = dmin_bits;
  return w;
}
inline Q6 make_q6(std::uint32_t n, std::uint32_t k, std::uint64_t seed, int scmax = 12,
           std::uint16_t d_bits = 0x3C00) {
  Lcg g{seed};
  Q6 w{n, k, std::vector<std::uint8_t>(std::size_t(n) * k), std::vector<std::int8_t>(std::size_t(n) * k / 16)};
  for (auto& v : w.q) v = std::uint8_t(g.range(0, 63));
  for (auto& v : w.sc) v = std::int8_t(g.range(-scmax, scmax));
  w.d = d_bits;
  return w;
}

// 16 metadata bytes of one super-block: fp16 d, dmin (1.0) and the 12-byte
// 6-bit scale/min packing (llama.cpp get_scale_min_k4 inverse).
inline void q4_meta(Q4 const& w, std::uint32_t r, std::uint32_t kb, std::uint8_t* m) {
  m[0] = std::uint8_t(w.d & 255); m[1] = std::uint8_t(w.d >> 8);
  m[2] = std::uint8_t(w.dmin & 255); m[3] = std::uint8_t(w.dmin >> 8);
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
inline void pack_020d(Q4 const& w, std::vector<std::uint8_t>& codes, std::vector<std::uint8_t>& meta) {
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
inline std::vector<std::uint8_t> ggml_q4(Q4 const& w) {
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
inline std::vector<std::uint8_t> ggml_q6(Q6 const& w) {
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
      y[208] = std::uint8_t(w.d & 255);
      y[209] = std::uint8_t(w.d >> 8);
    }
  return out;
}

}  // namespace fixture
