// C++ API test of the qw38::cuda interfaces (cuda/q4k_q8.hpp, decode_mmv.hpp,
// prefill.hpp and the runtime handles) on this build, in the style of the
// reference's tests/q4k_q8_test.cpp and tests/decode_mmv_unit_test.cpp:
// deterministic fixtures, closed-form checks computed here in double, typed
// rejections, graph capture with replays checked against eager results.
// Run: qw38_api_test [--list]; prints one line per check, exits nonzero on
// any failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "cuda/activation.hpp"
#include "cuda/alloc.hpp"
#include "cuda/buffer.hpp"
#include "cuda/copy.hpp"
#include "cuda/decode_mmv.hpp"
#include "cuda/event.hpp"
#include "cuda/fp8.hpp"
#include "cuda/nvfp4.hpp"
#include "cuda/graph.hpp"
#include "cuda/prefill.hpp"
#include "cuda/q4k_q8.hpp"
#include "cuda/stream.hpp"
#include "cuda/upload.hpp"

using namespace qw38::cuda;

namespace {

int g_failures = 0;

void expect(bool ok, std::string const& what) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  if (!ok) ++g_failures;
}

template <class T>
T unwrap(expected<T, Error> r, char const* what) {
  if (!r) {
    std::printf("FAIL %s: %s\n", what, error_message(r.error()).c_str());
    std::fflush(stdout);
    std::exit(2);
  }
  return std::move(*r);
}

void must(expected<void, Error> r, char const* what) {
  if (!r) {
    std::printf("FAIL %s: %s\n", what, error_message(r.error()).c_str());
    std::fflush(stdout);
    std::exit(2);
  }
}

// ---- scalar helpers ------------------------------------------------------------
float half_to_float(std::uint16_t h) {
  const int e = (h >> 10) & 31, m = h & 1023;
  const float v = e == 0 ? std::ldexp(float(m), -24) : std::ldexp(float(1024 + m), e - 25);
  return (h & 0x8000) ? -v : v;
}
std::uint16_t float_to_bf16(float f) {
  std::uint32_t u;
  std::memcpy(&u, &f, 4);
  if (((u >> 23) & 0xff) == 0xff) return std::uint16_t((u >> 16) | ((u & 0x7fffff) ? 0x40 : 0));
  return std::uint16_t((u + 0x7fff + ((u >> 16) & 1)) >> 16);
}
float bf16_to_float(std::uint16_t h) {
  std::uint32_t u = std::uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
void scale_min(std::uint8_t const* p, int g, int& s, int& m) {  // p = metadata bytes 4..15
  if (g < 4) {
    s = p[g] & 63;
    m = p[g + 4] & 63;
  } else {
    s = (p[g + 4] & 15) | ((p[g - 4] >> 6) << 4);
    m = (p[g + 4] >> 4) | ((p[g] >> 6) << 4);
  }
}

// ---- the reference test's odd-shape Q4_K fixture (tests/q4k_q8_test.cpp:36-60) ----
struct LogicalQ4K {
  std::uint32_t n, k, pk;
  std::vector<std::uint8_t> codes;  // [n][pk]
  std::vector<std::uint8_t> meta;   // [n][pk/256][16]
};

LogicalQ4K fixture_weight() {
  LogicalQ4K w{137, 259, 512, {}, {}};
  w.codes.assign(std::size_t(w.n) * w.pk, 0);
  w.meta.assign(std::size_t(w.n) * 2 * 16, 0);
  for (std::uint32_t r = 0; r < w.n; ++r) {
    for (std::uint32_t c = 0; c < w.k; ++c) w.codes[r * w.pk + c] = (r * 7 + c * 11) % 16;
    for (int b = 0; b < 2; ++b) {
      static constexpr unsigned kD[3] = {0x1400, 0x1800, 0x1A00};
      const unsigned dh = r == 0 ? 1 : kD[r % 3];
      const unsigned mh = r == 0 ? 2 : (b == 0 ? 0x1000 : 0x1400);
      std::uint8_t* m = &w.meta[(r * 2 + b) * 16];
      m[0] = dh & 255; m[1] = dh >> 8; m[2] = mh & 255; m[3] = mh >> 8;
      std::uint8_t* p = m + 4;
      for (int g = 0; g < 8; ++g) {
        const int s = (r * 13 + g * 17 + 3) % 64, mn = (r * 11 + g * 7 + 5) % 64;
        if (g < 4) {
          p[g] |= s;
          p[g + 4] |= mn;
        } else {
          p[g + 4] |= (s & 15) | ((mn & 15) << 4);
          p[g - 4] |= (s >> 4) << 6;
          p[g] |= (mn >> 4) << 6;
        }
      }
    }
  }
  return w;
}

// 0x020D tiles: tile row ((row/8)*kbs + kb)*8 + row%8; 128 B sequential
// nibbles and 16 B metadata per tile row.
void pack_020d(LogicalQ4K const& w, std::vector<std::byte>& codes, std::vector<std::byte>& meta) {
  const std::uint32_t pn = (w.n + 7) / 8 * 8, kbs = w.pk / 256;
  codes.assign(std::size_t(pn) * w.pk / 2, std::byte{0});
  meta.assign(std::size_t(pn) * kbs * 16, std::byte{0});
  for (std::uint32_t r = 0; r < w.n; ++r)
    for (std::uint32_t kb = 0; kb < kbs; ++kb) {
      const std::size_t tr = (std::size_t(r / 8) * kbs + kb) * 8 + r % 8;
      for (int j = 0; j < 128; ++j) {
        const std::uint8_t* c = &w.codes[r * w.pk + kb * 256 + 2 * j];
        codes[tr * 128 + j] = std::byte(c[0] | (c[1] << 4));
      }
      std::memcpy(&meta[tr * 16], &w.meta[(r * kbs + kb) * 16], 16);
    }
}

std::vector<std::uint16_t> fixture_input(std::uint32_t m, std::uint32_t k) {
  std::vector<std::uint16_t> x(std::size_t(m) * k);
  const float head[5] = {127.f, 0.5f, 1.5f, -0.5f, -1.5f};
  for (std::uint32_t r = 0; r < m; ++r)
    for (std::uint32_t c = 0; c < k; ++c) {
      float v = float(int((r * 23 + c * 19) % 67) - 44) * 0.125f * float(1 + r % 5);
      if (c >= 32 && c < 64) v = 0.f;
      if (c < 5) v = head[c];
      if (r == 2) v = 0.f;
      x[std::size_t(r) * k + c] = float_to_bf16(v);
    }
  return x;
}

// Closed-form Q8 pack of one 32-wide group (tests/q4k_q8_test.cpp:83-94).
void pack_group(float const* x, int n, std::int8_t* z, float& a, std::int32_t& sum) {
  float peak = 0.f;
  for (int i = 0; i < n; ++i) peak = std::fmax(peak, std::fabs(x[i]));
  a = peak == 0.f ? 1.f : peak / 127.f;
  sum = 0;
  for (int i = 0; i < 32; ++i) {
    float q = i < n ? std::nearbyint(x[i] / a) : 0.f;
    q = std::fmin(127.f, std::fmax(-127.f, q));
    z[i] = std::int8_t(q);
    sum += z[i];
  }
}

// out[t][r] in double: sum_g a_tg (d s_g dot - dmin m_g sum_tg)
std::vector<double> contract(LogicalQ4K const& w, std::vector<std::int8_t> const& z,
                             std::vector<float> const& a, std::vector<std::int32_t> const& su,
                             std::uint32_t m) {
  const std::uint32_t groups = w.pk / 32;
  std::vector<double> out(std::size_t(m) * w.n);
  for (std::uint32_t t = 0; t < m; ++t)
    for (std::uint32_t r = 0; r < w.n; ++r) {
      double acc = 0;
      for (std::uint32_t g = 0; g < groups; ++g) {
        const std::uint8_t* mb = &w.meta[(r * (w.pk / 256) + g / 8) * 16];
        int s, mn;
        scale_min(mb + 4, int(g % 8), s, mn);
        const double d = half_to_float(std::uint16_t(mb[0] | (mb[1] << 8)));
        const double dm = half_to_float(std::uint16_t(mb[2] | (mb[3] << 8)));
        long dot = 0;
        for (int i = 0; i < 32; ++i)
          dot += long(w.codes[r * w.pk + g * 32 + i]) * z[(std::size_t(t) * groups + g) * 32 + i];
        acc += double(a[t * groups + g]) * (d * s * double(dot) - dm * mn * double(su[t * groups + g]));
      }
      out[std::size_t(t) * w.n + r] = acc;
    }
  return out;
}

struct Dev {
  DeviceBuffer buf;
  template <class T>
  T* as() { return static_cast<T*>(buf.data()); }
};

template <class T>
Dev to_device(std::vector<T> const& v, Stream const& s) {
  auto b = unwrap(upload(std::as_bytes(std::span<T const>(v)), s), "upload");
  return Dev{std::move(b)};
}

template <class T>
std::vector<T> to_host(void const* p, std::size_t n, Stream const& s) {
  std::vector<T> v(n);
  must(copy_d2h(v.data(), p, n * sizeof(T), s), "copy_d2h");
  must(s.sync(), "sync");
  return v;
}

PrefillWeight weight_view(Dev& codes, Dev& meta, std::uint32_t n, std::uint32_t k) {
  PrefillWeight w;
  w.codes = codes.buf.data();
  w.scales = meta.buf.data();
  w.layout = kDecodeLayoutQ4KCandidateV2;
  w.quantizer = kDecodeQuantizerQ4KCandidateV2;
  w.n = n;
  w.k = k;
  w.padded_n = std::uint32_t(decode_pad_n(n));
  w.padded_k = decode_pad_k(k);
  w.codes_bytes = codes.buf.bytes();
  w.scales_bytes = meta.buf.bytes();
  return w;
}

// ---- tests ---------------------------------------------------------------------
void test_runtime(Stream const& s) {
  const auto before = malloc_count();
  {
    auto b = unwrap(DeviceBuffer::allocate(4096), "allocate");
    expect(malloc_count() == before + 1 && live_bytes() >= 4096, "DeviceBuffer counts its allocation");
    must(fill_pattern(b.data(), 4096, 7, s), "fill_pattern");
    auto h = to_host<std::uint8_t>(b.data(), 4096, s);
    bool ok = true;
    for (int i = 0; i < 4096; ++i) ok &= h[i] == std::uint8_t(7 + i);
    expect(ok, "fill_pattern writes seed + i");
    must(zero(b, s), "zero");
    h = to_host<std::uint8_t>(b.data(), 4096, s);
    ok = true;
    for (auto v : h) ok &= v == 0;
    expect(ok, "zero clears with a fill kernel");
  }
  expect(free_count() >= 1 && !DeviceBuffer::allocate(0), "empty allocation rejected");
  expect(!upload({}, s), "empty upload rejected");
  auto e0 = unwrap(Event::create_timing(), "event");
  auto e1 = unwrap(Event::create_timing(), "event");
  must(e0.record(s), "record");
  must(e1.record(s), "record");
  must(e1.sync(), "event sync");
  auto ms = elapsed_ms(e0, e1);
  expect(ms && *ms >= 0.f, "elapsed_ms between recorded events");
  testing::fail_next_stream_sync();
  expect(!s.sync(), "injected stream-sync failure is reported");
  expect(s.sync().has_value(), "next sync succeeds again");
}

void test_q4k_q8(Stream const& s) {
  const LogicalQ4K w = fixture_weight();
  std::vector<std::byte> codes, meta;
  pack_020d(w, codes, meta);
  auto dc = to_device(codes, s), dm = to_device(meta, s);
  const PrefillWeight pw = weight_view(dc, dm, w.n, w.k);
  const std::uint32_t ms[] = {1, 3, 8, 33, 127, 128, 129};
  std::vector<std::vector<float>> rows_m33;
  for (std::uint32_t m : ms) {
    const auto x = fixture_input(m, w.k);
    auto dx = to_device(x, s);
    const std::uint32_t groups = w.pk / 32;
    Dev codes_q{unwrap(DeviceBuffer::allocate(std::size_t(m) * w.pk), "alloc")};
    Dev scales_q{unwrap(DeviceBuffer::allocate(std::size_t(m) * groups * 4), "alloc")};
    Dev sums_q{unwrap(DeviceBuffer::allocate(std::size_t(m) * groups * 4), "alloc")};
    Dev flag{unwrap(DeviceBuffer::allocate(4), "alloc")};
    must(zero(flag.buf, s), "zero flag");
    Q8Input q{{codes_q.as<std::int8_t>(), std::size_t(m) * w.pk},
              {scales_q.as<float>(), std::size_t(m) * groups},
              {sums_q.as<std::int32_t>(), std::size_t(m) * groups},
              m, w.k, w.pk};
    must(pack_q8({dx.as<std::uint16_t>(), x.size()}, q, {flag.as<int>(), 1}, s), "pack_q8");
    // host closed form of the pack
    std::vector<std::int8_t> z(std::size_t(m) * w.pk);
    std::vector<float> a(std::size_t(m) * groups);
    std::vector<std::int32_t> su(std::size_t(m) * groups);
    for (std::uint32_t t = 0; t < m; ++t)
      for (std::uint32_t g = 0; g < groups; ++g) {
        float xs[32];
        const int n = int(std::min<std::uint32_t>(32, w.k > g * 32 ? w.k - g * 32 : 0));
        for (int i = 0; i < n; ++i) xs[i] = bf16_to_float(x[std::size_t(t) * w.k + g * 32 + i]);
        pack_group(xs, n, &z[(std::size_t(t) * groups + g) * 32], a[t * groups + g], su[t * groups + g]);
      }
    const auto gz = to_host<std::int8_t>(codes_q.buf.data(), z.size(), s);
    const auto ga = to_host<float>(scales_q.buf.data(), a.size(), s);
    const auto gs = to_host<std::int32_t>(sums_q.buf.data(), su.size(), s);
    expect(gz == z && std::memcmp(ga.data(), a.data(), a.size() * 4) == 0 && gs == su,
           "pack_q8 bit-exact against the closed form, m=" + std::to_string(m));
    Dev out{unwrap(DeviceBuffer::allocate(std::size_t(m) * w.n * 4), "alloc")};
    must(q4k_q8_project(pw, q, {out.as<float>(), std::size_t(m) * w.n}, s), "project");
    const auto y = to_host<float>(out.buf.data(), std::size_t(m) * w.n, s);
    const auto ref = contract(w, z, a, su, m);
    double rms = 0, maxerr = 0;
    for (std::size_t i = 0; i < ref.size(); ++i) {
      rms += ref[i] * ref[i];
      maxerr = std::fmax(maxerr, std::fabs(double(y[i]) - ref[i]));
    }
    rms = std::sqrt(rms / double(ref.size()));
    expect(maxerr <= 1e-3 * rms, "q4k_q8_project within 1e-3 rms of the closed form, m=" + std::to_string(m));
    if (m == 33 || m == 129) rows_m33.emplace_back(y.begin(), y.begin() + 33 * w.n);
  }
  expect(rows_m33.size() == 2 && rows_m33[0] == rows_m33[1],
         "MMQ token rows bitwise independent of the tiling (m=33 vs m=129)");
  // typed rejections before any launch
  PrefillWeight bad = pw;
  bad.quantizer = kDecodeQuantizerQ4G64V0;
  Q8Input empty_q{};
  auto r = q4k_q8_project(bad, empty_q, {}, s);
  expect(!r && r.error().code == ErrorCode::InvalidArgument, "mismatched quantizer rejected");
}

void test_decode_onehot(Stream const& s) {
  // tests/decode_mmv_unit_test.cpp:405-478 restated: each rebuilt BF16 operand
  // comes back exactly through a one-hot input.
  constexpr std::uint32_t n = 8, k = 256;
  const std::uint16_t d_bits[n] = {0, 1, 2, 0x3ff, 0x400, 0x1400, 0x2400, 0x3400};
  const std::uint16_t m_bits[n] = {0, 3, 1, 0x201, 0x3ff, 0x1000, 0x2000, 0x3000};
  std::vector<std::byte> codes(n * k / 2), meta(n * 16);
  std::vector<float> expected_w(n * k);
  for (std::uint32_t row = 0; row < n; ++row) {
    std::uint8_t* mt = reinterpret_cast<std::uint8_t*>(&meta[row * 16]);
    mt[0] = d_bits[row] & 255; mt[1] = d_bits[row] >> 8;
    mt[2] = m_bits[row] & 255; mt[3] = m_bits[row] >> 8;
    int sc[8], mn[8];
    for (int g = 0; g < 8; ++g) {
      sc[g] = (g * 9 + row * 13) % 64;
      mn[g] = (63 - g * 7 + row * 3) % 64;
    }
    for (int g = 0; g < 4; ++g) {
      mt[4 + g] = std::uint8_t(sc[g] | ((sc[g + 4] >> 4) << 6));
      mt[8 + g] = std::uint8_t(mn[g] | ((mn[g + 4] >> 4) << 6));
      mt[12 + g] = std::uint8_t((sc[g + 4] & 15) | ((mn[g + 4] & 15) << 4));
    }
    for (std::uint32_t col = 0; col < k; ++col) {
      const unsigned code = (col + 5 * row) % 16;
      codes[row * k / 2 + col / 2] |= std::byte(code << (4 * (col % 2)));
      const float d = half_to_float(d_bits[row]) * float(sc[col / 32]);
      const float m = half_to_float(m_bits[row]) * float(mn[col / 32]);
      volatile float prod = d * float(code);
      expected_w[row * k + col] = bf16_to_float(float_to_bf16(prod - m));
    }
  }
  auto dc = to_device(codes, s), dm = to_device(meta, s);
  Dev y{unwrap(DeviceBuffer::allocate(n * 4), "alloc")};
  Dev x{unwrap(DeviceBuffer::allocate(k * 2), "alloc")};
  DecodeMmvDesc d;
  d.layout = kDecodeLayoutQ4KCandidateV2;
  d.quantizer = kDecodeQuantizerQ4KCandidateV2;
  d.n = d.padded_n = n;
  d.k = d.padded_k = k;
  d.codes = decode_matrix_view(dc.buf.data(), DecodeDtype::Q4, d.layout, n, k, n, k,
                               dc.buf.bytes(), 16);
  d.scales = decode_matrix_view(dm.buf.data(), DecodeDtype::Fp16, d.layout, n, 8, n, 8,
                                dm.buf.bytes(), 2);
  d.input = decode_vector_view(x.buf.data(), DecodeDtype::Bf16, kDecodeLayoutBf16VectorV0, k, k * 2,
                               2, false);
  d.output = decode_vector_view(y.buf.data(), DecodeDtype::Fp32, kDecodeLayoutFp32VectorV0, n, n * 4,
                                4, true);
  d.epilogue = DecodeEpilogue::StoreFp32;
  bool all = true;
  for (std::uint32_t col = 0; col < k; ++col) {
    std::vector<std::uint16_t> xv(k, 0);
    xv[col] = 0x3f80;
    must(copy_h2d(x.buf.data(), xv.data(), k * 2, s), "copy");
    must(launch_decode_mmv(d, s), "decode_mmv");
    const auto got = to_host<float>(y.buf.data(), n, s);
    for (std::uint32_t row = 0; row < n; ++row) all &= got[row] == expected_w[row * k + col];
  }
  expect(all, "decode_mmv one-hot returns every rebuilt BF16 operand exactly");
  DecodeMmvDesc bad = d;
  bad.quantizer = kDecodeQuantizerQ4G64V0;
  expect(!launch_decode_mmv(bad, s), "decode_mmv: mismatched quantizer rejected");
  bad = d;
  bad.scales.bytes /= 2;
  expect(!launch_decode_mmv(bad, s), "decode_mmv: truncated metadata rejected");
  expect(!launch_decode_ab_bf16({d, d}, s), "decode_ab_bf16 rejects a layout other than BF16 dense tiles");
}

void test_graph_replay(Stream const& s) {
  // a captured projection replays with eager work and syncs in between and
  // matches the eager result every time
  const LogicalQ4K w = fixture_weight();
  std::vector<std::byte> codes, meta;
  pack_020d(w, codes, meta);
  auto dc = to_device(codes, s), dm = to_device(meta, s);
  const PrefillWeight pw = weight_view(dc, dm, w.n, w.k);
  const std::uint32_t m = 40, groups = w.pk / 32;
  const auto x = fixture_input(m, w.k);
  auto dx = to_device(x, s);
  Dev zq{unwrap(DeviceBuffer::allocate(std::size_t(m) * w.pk), "alloc")};
  Dev aq{unwrap(DeviceBuffer::allocate(std::size_t(m) * groups * 4), "alloc")};
  Dev sq{unwrap(DeviceBuffer::allocate(std::size_t(m) * groups * 4), "alloc")};
  Dev flag{unwrap(DeviceBuffer::allocate(4), "alloc")};
  must(zero(flag.buf, s), "zero");
  Q8Input q{{zq.as<std::int8_t>(), std::size_t(m) * w.pk}, {aq.as<float>(), std::size_t(m) * groups},
            {sq.as<std::int32_t>(), std::size_t(m) * groups}, m, w.k, w.pk};
  Dev out{unwrap(DeviceBuffer::allocate(std::size_t(m) * w.n * 4), "alloc")};
  std::span<float> os{out.as<float>(), std::size_t(m) * w.n};
  must(pack_q8({dx.as<std::uint16_t>(), x.size()}, q, {flag.as<int>(), 1}, s), "pack");
  must(q4k_q8_project(pw, q, os, s), "eager");
  const auto eager = to_host<float>(out.buf.data(), os.size(), s);
  auto g = unwrap(Graph::begin(s), "graph begin");
  must(pack_q8({dx.as<std::uint16_t>(), x.size()}, q, {flag.as<int>(), 1}, s), "capture pack");
  must(q4k_q8_project(pw, q, os, s), "capture project");
  must(g.finish(), "graph finish");
  bool ok = true;
  for (int rep = 0; rep < 3; ++rep) {
    must(zero(out.buf, s), "zero between replays");
    must(g.launch(s), "graph launch");
    ok &= to_host<float>(out.buf.data(), os.size(), s) == eager;
  }
  expect(ok, "graph replays match the eager projection (3 replays)");
  expect(require_uncaptured(s).has_value(), "stream is no longer capturing");
}

void test_prefill(Stream const& s) {
  auto engine = unwrap(PrefillEngine::create(s, 64, 512), "prefill create");
  expect(engine.workspace_bytes() > 0 && engine.token_capacity() == 64, "engine owns its workspace");
  expect(!PrefillEngine::create(s, 0), "zero capacity rejected");
  expect(!PrefillEngine::create(s, 64, 300), "invalid weight_rows rejected");
  // project the fixture weight (K = 512 logical for the BF16 path: k % 256 == 0)
  LogicalQ4K w = fixture_weight();
  w.k = 512;  // codes beyond 259 are zero in the fixture
  std::vector<std::byte> codes, meta;
  pack_020d(w, codes, meta);
  auto dc = to_device(codes, s), dm = to_device(meta, s);
  const PrefillWeight pw = weight_view(dc, dm, w.n, w.k);
  const std::uint32_t m = 20;
  const auto x = fixture_input(m, w.k);
  auto dx = to_device(x, s);
  Dev out{unwrap(DeviceBuffer::allocate(std::size_t(m) * w.n * 4), "alloc")};
  PrefillProjection p;
  p.weight = pw;
  p.input = dx.as<std::uint16_t>();
  p.output = out.buf.data();
  p.valid_tokens = m;
  p.epilogue = PrefillEpilogue::StoreFp32;
  must(engine.project(p), "prefill project");
  const auto y = to_host<float>(out.buf.data(), std::size_t(m) * w.n, s);
  double maxerr = 0, rms = 0;
  for (std::uint32_t t = 0; t < m; ++t)
    for (std::uint32_t r = 0; r < w.n; ++r) {
      double acc = 0;
      for (std::uint32_t c = 0; c < w.k; ++c) {
        const std::uint8_t* mb = &w.meta[(r * 2 + c / 256) * 16];
        int sc, mn;
        scale_min(mb + 4, int((c % 256) / 32), sc, mn);
        const float d = half_to_float(std::uint16_t(mb[0] | (mb[1] << 8))) * float(sc);
        const float dmn = half_to_float(std::uint16_t(mb[2] | (mb[3] << 8))) * float(mn);
        volatile float prod = d * float(w.codes[r * w.pk + c]);
        const float wv = bf16_to_float(float_to_bf16(prod - dmn));
        acc += double(wv) * bf16_to_float(x[std::size_t(t) * w.k + c]);
      }
      rms += acc * acc;
      maxerr = std::fmax(maxerr, std::fabs(acc - double(y[std::size_t(t) * w.n + r])));
    }
  rms = std::sqrt(rms / double(m * w.n));
  expect(maxerr <= 1e-3 * rms + 1e-6, "PrefillEngine::project matches the BF16 operand closed form");
  p.valid_tokens = 65;
  expect(!engine.project(p), "valid_tokens above capacity rejected");
  p.valid_tokens = m;
  p.epilogue = PrefillEpilogue::ResidualAddFp32;
  expect(!engine.project(p), "residual epilogue without residual rejected");
  std::uint32_t rows[2] = {1, 1};
  expect(!engine.head_evaluation(pw, dx.as<std::uint16_t>(), m, 0, rows, out.as<float>()),
         "head evaluation contract (shape, duplicates) rejected");
}

// OCP E4M3FN value of a code (bias 7, no infinities, 0x7F / 0xFF NaN).
double e4m3_value(std::uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  const double v = e == 0 ? std::ldexp(double(m), -9) : std::ldexp(double(8 + m), e - 10);
  return (c & 0x80) ? -v : v;
}

// The engine's FP8 consumers (tests/fp8_test.cpp:238-266): the M > 1 projection
// equals fp8_gemm on the engine-owned pack, siblings keep the pack, missing or
// incompatible packs are refused, and M = 1 runs decode equal to fp8_gemv.
void test_fp8(Stream const& s) {
  constexpr unsigned n = 128, k = 5120, m = 256;
  auto engine = unwrap(PrefillEngine::create(s, m, 512, PrefillDispatch::BoundedUnpackBf16Cublas, true),
                       "FP8 engine create");
  const int sm = unwrap(prepare_fp8_gemm(s), "prepare_fp8_gemm");
  expect(sm > 0, "prepare_fp8_gemm reports the device's compute units");
  const Fp8Input op = engine.fp8_operand(m, k);
  expect(op.m == m && op.k == k && op.codes.size() == std::size_t(m) * k &&
             op.scales.size() == std::size_t(m) * (k / 128),
         "fp8_operand spans the engine-owned pack");
  expect(engine.fp8_operand(m + 1, k).codes.empty() && engine.fp8_operand(m, 6272).codes.empty(),
         "fp8_operand refuses shapes beyond capacity");
  std::vector<std::uint8_t> wc(std::size_t(n) * k);
  for (std::size_t i = 0; i < wc.size(); ++i) {
    std::uint8_t c = std::uint8_t((i * 37 + i / k * 11) & 0xff);
    wc[i] = (c & 0x7f) == 0x7f ? 0 : c;
  }
  std::vector<float> ws(k / 128);
  for (unsigned b = 0; b < ws.size(); ++b) ws[b] = std::ldexp(1.0f + float(b % 5) / 8, -9 - int(b % 3));
  std::vector<std::uint16_t> x(std::size_t(m) * k);
  for (unsigned t = 0; t < m; ++t)
    for (unsigned c = 0; c < k; ++c)
      x[std::size_t(t) * k + c] =
          float_to_bf16(float(int((t * 23 + c * 17) % 97) - 48) * 0.03125f * float(1 + t % 3));
  auto dwc = to_device(wc, s), dws = to_device(ws, s), dx = to_device(x, s);
  must(pack_fp8({dx.as<std::uint16_t>(), x.size()}, m, k,
                {const_cast<std::uint8_t*>(op.codes.data()), op.codes.size()},
                {const_cast<float*>(op.scales.data()), op.scales.size()}, s),
       "pack_fp8 into the engine operand");
  const Fp8Weight fw{{dwc.as<std::uint8_t>(), wc.size()}, {dws.as<float>(), ws.size()}, n, k};
  const PrefillWeight pw{dwc.buf.data(), dws.buf.data(), kDecodeLayoutFp8V1, kDecodeQuantizerFp8V1,
                         n, k, n, k, wc.size(), ws.size() * 4};
  Dev projected{unwrap(DeviceBuffer::allocate(std::size_t(m) * n * 4), "alloc")};
  Dev reference{unwrap(DeviceBuffer::allocate(std::size_t(m) * n * 4), "alloc")};
  Dev work{unwrap(DeviceBuffer::allocate(4096), "alloc")};
  PrefillProjection p{.weight = pw, .input = dx.as<std::uint16_t>(), .output = projected.buf.data(),
                      .valid_tokens = m, .epilogue = PrefillEpilogue::StoreFp32, .packed = op};
  must(engine.project(p), "FP8 engine project");
  must(fp8_gemm(fw, op, {reference.as<float>(), std::size_t(m) * n},
                {static_cast<std::byte*>(work.buf.data()), 4096}, sm, s),
       "fp8_gemm");
  const auto result = to_host<float>(projected.buf.data(), std::size_t(m) * n, s);
  expect(result == to_host<float>(reference.buf.data(), std::size_t(m) * n, s),
         "FP8 prefill projection equals fp8_gemm on the same pack");
  // closed form in double on the pack actually used
  const auto pc = to_host<std::uint8_t>(op.codes.data(), op.codes.size(), s);
  const auto psc = to_host<float>(op.scales.data(), op.scales.size(), s);
  bool close = true;
  for (unsigned t : {0u, 1u, 131u, 255u})
    for (unsigned r = 0; r < n; r += 9) {
      double acc = 0, l1 = 0;
      for (unsigned c = 0; c < k; ++c) {
        const double a = e4m3_value(pc[std::size_t(t) * k + c]) * psc[std::size_t(c / 128) * m + t];
        const double b = e4m3_value(wc[std::size_t(r) * k + c]) * ws[c / 128];
        acc += a * b;
        l1 += std::fabs(a * b);
      }
      close &= std::fabs(acc - result[std::size_t(t) * n + r]) < 1e-4 + 1e-5 * l1;
    }
  expect(close, "FP8 projection within 1e-4 + 1e-5 * l1 of the double contraction");
  must(engine.project(p), "FP8 sibling project");
  expect(result == to_host<float>(projected.buf.data(), std::size_t(m) * n, s),
         "a sibling consumer preserves the pack");
  p.packed = {};
  expect(!engine.project(p), "consumer refuses a missing pack");
  p.packed = op;
  p.packed.k = 6144;
  expect(!engine.project(p), "consumer refuses an incompatible pack");
  p.packed = {};
  p.valid_tokens = 1;
  must(engine.project(p), "FP8 decode project");
  must(fp8_gemv(fw, {dx.as<std::uint16_t>(), k}, {reference.as<float>(), n}, s), "fp8_gemv");
  const auto one = to_host<float>(projected.buf.data(), n, s), ref = to_host<float>(reference.buf.data(), n, s);
  expect(one == ref, "M = 1 decode equals fp8_gemv on the same view");
  p.packed = op;
  expect(!engine.project(p), "M = 1 refuses an unused decode pack");
}

// NVFP4 weight from BF16 rows: packed like an activation, behind a 256-byte
// header that holds the FP32 global factor 1.
struct Nvfp4W {
  Dev codes, scales;
  PrefillWeight view;
};
Nvfp4W nvfp4_weight(unsigned n, unsigned k, unsigned seed, Stream const& s) {
  std::vector<std::uint16_t> w(std::size_t(n) * k);
  for (std::size_t i = 0; i < w.size(); ++i)
    w[i] = float_to_bf16(float(int((i * 29 + seed * 7 + i / k * 3) % 61) - 30) / 16.0f);
  auto dw = to_device(w, s);
  const std::uint64_t cb = std::uint64_t(n) * k / 2, sb = (n + 127) / 128 * 128ull * (k / 16);
  std::vector<std::uint8_t> hdr(256 + sb, 0);
  const float one = 1.0f;
  std::memcpy(hdr.data(), &one, 4);
  Nvfp4W r{Dev{unwrap(DeviceBuffer::allocate(cb), "alloc")}, to_device(hdr, s), {}};
  must(launch_pack_nvfp4(dw.as<std::uint16_t>(), r.codes.as<std::uint8_t>(), r.scales.as<std::uint8_t>() + 256,
                         n, k, s),
       "pack NVFP4 weight");
  r.view = PrefillWeight{r.codes.buf.data(), r.scales.buf.data(), kDecodeLayoutNvFp4V1,
                         kDecodeQuantizerNvFp4V1, n, k, n, k, cb, 256 + sb};
  return r;
}

void test_nvfp4(Stream const& s) {
  constexpr unsigned n = 136, k = 5120, m = 77;
  auto engine = unwrap(PrefillEngine::create(s, 128, 512), "NVFP4 engine create");
  const int sm = unwrap(prepare_nvfp4_gemm(128, 0, s), "prepare_nvfp4_gemm");
  expect(sm > 0, "prepare_nvfp4_gemm reports the device's compute units");
  auto gate = nvfp4_weight(n, k, 1, s), up = nvfp4_weight(n, k, 2, s);
  std::vector<std::uint16_t> x(std::size_t(m) * k);
  for (std::size_t i = 0; i < x.size(); ++i)
    x[i] = float_to_bf16(float(int((i * 17 + 5) % 131) - 65) / 27.0f);
  auto dx = to_device(x, s);
  // the engine's NVFP4 projection equals pack + nvfp4_gemm_tile
  Dev proj{unwrap(DeviceBuffer::allocate(std::size_t(m) * n * 4), "alloc")};
  PrefillProjection p{.weight = gate.view, .input = dx.as<std::uint16_t>(), .output = proj.buf.data(),
                      .valid_tokens = m, .epilogue = PrefillEpilogue::StoreFp32};
  must(engine.project(p), "NVFP4 engine project");
  Dev xc{unwrap(DeviceBuffer::allocate(std::size_t(m) * k / 2), "alloc")};
  Dev xs{unwrap(DeviceBuffer::allocate(std::size_t(128) * (k / 16)), "alloc")};
  must(launch_pack_nvfp4(dx.as<std::uint16_t>(), xc.as<std::uint8_t>(), xs.as<std::uint8_t>(), m, k, s),
       "pack NVFP4 activations");
  Dev g{unwrap(DeviceBuffer::allocate(std::size_t(m) * n * 4), "alloc")};
  Dev u{unwrap(DeviceBuffer::allocate(std::size_t(m) * n * 4), "alloc")};
  must(nvfp4_gemm_tile(gate.view.codes, gate.view.scales, xc.as<std::uint8_t>(), xs.as<std::uint8_t>(), m, n,
                       k, 0, g.as<float>(), nullptr, 0, sm, s),
       "nvfp4_gemm_tile gate");
  must(nvfp4_gemm_tile(up.view.codes, up.view.scales, xc.as<std::uint8_t>(), xs.as<std::uint8_t>(), m, n, k,
                       0, u.as<float>(), nullptr, 0, sm, s),
       "nvfp4_gemm_tile up");
  const auto yp = to_host<float>(proj.buf.data(), std::size_t(m) * n, s);
  const auto yg = to_host<float>(g.buf.data(), std::size_t(m) * n, s);
  const auto yu = to_host<float>(u.buf.data(), std::size_t(m) * n, s);
  expect(yp == yg, "NVFP4 engine projection equals pack + nvfp4_gemm_tile bitwise");
  // paired SwiGLU: BF16(SiLU(gate) * up) of the same two tiles, within one BF16 ulp
  Dev sw{unwrap(DeviceBuffer::allocate(std::size_t(m) * n * 2), "alloc")};
  must(engine.paired_swiglu(gate.view, up.view, dx.as<std::uint16_t>(), sw.as<std::uint16_t>(), m, 0),
       "NVFP4 paired SwiGLU");
  const auto ys = to_host<std::uint16_t>(sw.buf.data(), std::size_t(m) * n, s);
  bool close = true;
  for (std::size_t i = 0; i < ys.size(); ++i) {
    const double gv = yg[i], want = gv / (1.0 + std::exp(-gv)) * yu[i];
    const std::uint16_t wb = float_to_bf16(float(want));
    close &= std::abs(int(ys[i]) - int(wb)) <= 1;
  }
  expect(close, "NVFP4 paired SwiGLU within one BF16 ulp of SiLU(gate) * up");
  // a Q4_K down projection is not an NVFP4 pair partner
  PrefillWeight mixed = up.view;
  mixed.layout = 0x020D;
  expect(!engine.paired_swiglu(gate.view, mixed, dx.as<std::uint16_t>(), sw.as<std::uint16_t>(), m, 0),
         "NVFP4 gate with a non-NVFP4 up rejected");
}

}  // namespace

int main(int argc, char** argv) {
  const char* names[] = {"runtime", "q4k_q8", "decode_onehot", "graph_replay", "prefill", "fp8", "nvfp4"};
  if (argc > 1 && std::strcmp(argv[1], "--list") == 0) {
    for (auto* n : names) std::printf("%s\n", n);
    return 0;
  }
  auto stream = unwrap(Stream::create(), "stream");
  std::printf("== runtime\n");
  test_runtime(stream);
  std::printf("== q4k_q8\n");
  test_q4k_q8(stream);
  std::printf("== decode_onehot\n");
  test_decode_onehot(stream);
  std::printf("== graph_replay\n");
  test_graph_replay(stream);
  std::printf("== prefill\n");
  test_prefill(stream);
  std::printf("== fp8\n");
  test_fp8(stream);
  std::printf("== nvfp4\n");
  test_nvfp4(stream);
  must(stream.sync(), "final sync");
  std::printf("%d failure(s)\n", g_failures);
  return g_failures == 0 ? 0 : 1;
}
