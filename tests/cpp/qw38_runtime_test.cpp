// Runtime callers of the projection path over an uploaded `.qw38` model (the
// reference's tests/mlp_integration_test.cpp, q8_mlp_integration_test.cpp and
// the decode-token graph of runtime/language_model.cpp cover the same
// contracts): two MLP layers 5120 -> 17408 -> 5120, layer 0 in the reference
// layout 0x020D, layer 1 as GGML-order Q4_K gate/up (repacked to 0x0240 at
// load) and a GGML-order Q6_K down projection (repacked to 0x0241).
//
// Checks: the plan's Q8 route equals a direct q4k_q8_mlp call bitwise; the
// BF16 route's stages match the oracle's BF16 GEMV (oracle/liboracle.so, test
// infrastructure) within the north-star tolerance; a
// decode token captured in a hipGraph and replayed for several tokens equals
// the eager submission bitwise, replay after replay; a nonfinite activation
// is reported by complete_unit and poisons the session; prefill chunks (Q8
// route and PrefillEngine route) equal their direct calls; capture is
// rejected by the public synchronous entry points.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "artifact_fixture.hpp"
#include "oracle.h"
#include "cuda/buffer.hpp"
#include "cuda/copy.hpp"
#include "cuda/graph.hpp"
#include "cuda/prefill.hpp"
#include "cuda/q4k_q8.hpp"
#include "cuda/stream.hpp"
#include "runtime/mlp.hpp"
#include "runtime/model.hpp"

namespace F = qw38::format;
namespace R = qw38::runtime;
using namespace qw38::cuda;
using namespace fixture;

namespace {

int g_failures = 0;
void expect(bool ok, std::string const& what) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  std::fflush(stdout);
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

std::uint16_t bf16(float f) {
  std::uint32_t u;
  std::memcpy(&u, &f, 4);
  return std::uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

std::vector<float> uniform(std::size_t n, std::uint64_t seed, float scale) {
  Lcg g{seed};
  std::vector<float> v(n);
  for (auto& x : v) x = scale * (float(g.next() % 200001u) / 100000.f - 1.f);
  return v;
}

std::vector<std::uint8_t> gamma_bytes(std::uint64_t seed) {
  const auto g = uniform(R::kHidden, seed, 0.2f);
  std::vector<std::uint8_t> out(R::kHidden * 2);
  for (std::uint32_t i = 0; i < R::kHidden; ++i) {
    const std::uint16_t b = bf16(g[i]);
    out[2 * i] = std::uint8_t(b & 255);
    out[2 * i + 1] = std::uint8_t(b >> 8);
  }
  return out;
}

float bf16_value(std::uint16_t b) {
  const std::uint32_t u = std::uint32_t(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Layer-0 weights as build_artifact() makes them (ids 1, 2, 3: gate, up, down).
Q4 layer0_weight(int i) {
  const std::uint32_t n = i == 2 ? R::kHidden : R::kFfnWidth, k = i == 2 ? R::kFfnWidth : R::kHidden;
  return make_q4(n, k, 100 + 1 + i, 63, 0x1800, 0x1400);
}

// The oracle's BF16-operand GEMV (float64 sums) of a logical Q4_K weight.
std::vector<double> oracle_bf16_gemv(Q4 const& w, std::vector<std::uint16_t> const& x) {
  const std::uint32_t kbs = w.k / 256;
  std::vector<std::uint8_t> meta(std::size_t(w.n) * kbs * 16);
  for (std::uint32_t r = 0; r < w.n; ++r)
    for (std::uint32_t kb = 0; kb < kbs; ++kb) q4_meta(w, r, kb, &meta[(std::size_t(r) * kbs + kb) * 16]);
  std::vector<double> out(w.n);
  orc_q4k_bf16_gemv(w.c.data(), meta.data(), w.n, w.k, w.k, x.data(), out.data(), 0);
  return out;
}

std::string name(int layer, char const* suffix) {
  return "model.language_model.layers." + std::to_string(layer) + suffix;
}

std::vector<std::uint8_t> build_artifact() {
  std::vector<WTensor> ts;
  std::uint32_t id = 1;
  // layer 0: 0x020D tiles, as the reference compiler emits them
  for (auto [suffix, n, k] : {std::tuple{".mlp.gate_proj.weight", R::kFfnWidth, R::kHidden},
                              std::tuple{".mlp.up_proj.weight", R::kFfnWidth, R::kHidden},
                              std::tuple{".mlp.down_proj.weight", R::kHidden, R::kFfnWidth}}) {
    const Q4 w = make_q4(n, k, 100 + id, 63, 0x1800, 0x1400);
    std::vector<std::uint8_t> co, mo;
    pack_020d(w, co, mo);
    ts.push_back({id++, name(0, suffix), n, k, 0x0001, F::kQuantizerQ4K, F::kLayoutQ4KTiles, co, mo});
  }
  ts.push_back({id++, name(0, ".post_attention_layernorm.weight"), R::kHidden, 1, 0x0003, 0x0100, 0x0205,
                gamma_bytes(7), {}});
  // layer 1: GGML-order blocks, repacked at load
  for (auto [suffix, n, k] : {std::tuple{".mlp.gate_proj.weight", R::kFfnWidth, R::kHidden},
                              std::tuple{".mlp.up_proj.weight", R::kFfnWidth, R::kHidden}}) {
    const Q4 w = make_q4(n, k, 200 + id, 63, 0x1800, 0x1400);
    ts.push_back({id++, name(1, suffix), n, k, 0x0001, F::kQuantizerQ4K, F::kLayoutQ4KGgmlBlocks, ggml_q4(w), {}});
  }
  {
    const Q6 w = make_q6(R::kHidden, R::kFfnWidth, 300, 100, 0x1000);
    ts.push_back({id++, name(1, ".mlp.down_proj.weight"), R::kHidden, R::kFfnWidth, 0x0002, F::kQuantizerQ6K,
                  F::kLayoutQ6KGgmlBlocks, ggml_q6(w), {}});
  }
  ts.push_back({id++, name(1, ".post_attention_layernorm.weight"), R::kHidden, 1, 0x0003, 0x0100, 0x0205,
                gamma_bytes(8), {}});
  return write_artifact(ts, {});
}

struct Dev {
  DeviceBuffer b;
  template <class T>
  T* as() { return static_cast<T*>(b.data()); }
};
Dev alloc(std::uint64_t bytes, Stream const& s) { return Dev{unwrap(DeviceBuffer::allocate(bytes, s.device()), "alloc")}; }
template <class T>
void put(Dev& d, std::vector<T> const& v, Stream const& s) {
  must(copy_h2d(d.b.data(), v.data(), v.size() * sizeof(T), s), "copy_h2d");
}
template <class T>
std::vector<T> get(Dev const& d, std::size_t n, Stream const& s) {
  std::vector<T> v(n);
  must(copy_d2h(v.data(), d.b.data(), n * sizeof(T), s), "copy_d2h");
  must(s.sync(), "sync");
  return v;
}

bool same_bits(std::vector<float> const& a, std::vector<float> const& b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * 4) == 0;
}

// max |a - b| relative to rms(b)
double rel_dev(std::vector<float> const& a, std::vector<float> const& b) {
  double mx = 0, ss = 0;
  for (std::size_t i = 0; i < a.size(); ++i) {
    mx = std::max(mx, std::fabs(double(a[i]) - double(b[i])));
    ss += double(b[i]) * b[i];
  }
  return mx / std::sqrt(ss / double(b.size()) + 1e-30);
}

void run(Stream const& s) {
  const auto bytes = build_artifact();
  auto art = F::Artifact::parse(std::as_bytes(std::span(bytes)));
  if (!art) { expect(false, "parse: " + F::error_message(art.error())); return; }
  auto model = unwrap(R::Model::upload(*art, s), "Model::upload");
  auto session = unwrap(R::Session::create(s, 64), "Session::create");
  const std::uint32_t H = R::kHidden, Fw = R::kFfnWidth;

  Dev h_mid = alloc(64ull * H * 4, s), next_h = alloc(64ull * H * 4, s), ref = alloc(64ull * H * 4, s);
  Dev normalized = alloc(H * 2, s), swiglu = alloc(Fw * 2, s);
  Dev ws = alloc(q8_mlp_workspace_bytes(64), s);
  R::MlpBuffers io{h_mid.as<float>(), next_h.as<float>(), normalized.as<std::uint16_t>(), swiglu.as<std::uint16_t>()};

  for (int layer = 0; layer < 2; ++layer) {
    auto plan = unwrap(R::bind_mlp_plan(model, session, layer, s, io), "bind Q8");
    put(h_mid, uniform(H, 11 + layer, 2.f), s);
    must(R::execute_decode_mlp(plan), "execute_decode_mlp");
    const auto y = get<float>(next_h, H, s);
    bool submitted = false;
    must(q4k_q8_mlp(plan.gate, plan.up, plan.down, h_mid.as<float>(), plan.gamma, plan.eps, ref.as<float>(), 1,
                    {ws.b.as_bytes(), std::size_t(ws.b.bytes())}, s, submitted),
         "direct q4k_q8_mlp");
    const auto yr = get<float>(ref, H, s);
    expect(same_bits(y, yr), "layer " + std::to_string(layer) + ": Q8 route equals a direct q4k_q8_mlp bitwise");
    bool finite = true;
    for (float v : y) finite = finite && std::isfinite(v);
    expect(finite, "layer " + std::to_string(layer) + ": decode MLP output finite");
  }
  {
    // BF16 route (0x020D layer only) stage by stage against the oracle's BF16
    // GEMV (orc_q4k_bf16_gemv: cuda/decode_mmv.cu:121-140 restated, float64
    // sums) on the same weights and on the route's own BF16 intermediates:
    // the paired gate/up SwiGLU store within one BF16 ulp of BF16(SiLU(g)*u)
    // from the oracle's g and u, and the down projection + residual within
    // the north-star tolerance (max |y - ref| <= 1e-3 rms(ref), mean relative
    // error <= 1e-5).
    auto p16 = unwrap(R::bind_mlp_plan(model, session, 0, s, io, R::MlpRoute::Bf16), "bind BF16");
    const auto x = uniform(H, 21, 2.f);
    put(h_mid, x, s);
    must(R::execute_decode_mlp(p16), "BF16");
    const auto y16 = get<float>(next_h, H, s);
    const auto nb = get<std::uint16_t>(normalized, H, s);
    const auto sw = get<std::uint16_t>(swiglu, Fw, s);
    const Q4 wg = layer0_weight(0), wu = layer0_weight(1), wd = layer0_weight(2);
    const auto g = oracle_bf16_gemv(wg, nb), u = oracle_bf16_gemv(wu, nb), dn = oracle_bf16_gemv(wd, sw);
    double rms_sw = 0;
    std::vector<double> want_sw(Fw);
    for (std::uint32_t i = 0; i < Fw; ++i) {
      const float gf = float(g[i]), uf = float(u[i]);
      want_sw[i] = double(bf16_value(bf16(gf / (1.0f + orc_expf(-gf)) * uf)));
      rms_sw += want_sw[i] * want_sw[i];
    }
    rms_sw = std::sqrt(rms_sw / Fw);
    bool sw_ok = true;
    for (std::uint32_t i = 0; i < Fw; ++i)
      sw_ok = sw_ok && std::fabs(double(bf16_value(sw[i])) - want_sw[i]) <= std::ldexp(std::fabs(want_sw[i]), -7) + 1e-6 * rms_sw;
    expect(sw_ok, "BF16 route: paired gate/up SwiGLU store within one BF16 ulp of the oracle's BF16 GEMVs");
    std::vector<double> want_y(H);
    for (std::uint32_t i = 0; i < H; ++i) want_y[i] = double(x[i]) + dn[i];
    double mx = 0, ss = 0, sa = 0, sr = 0;
    for (std::uint32_t i = 0; i < H; ++i) {
      const double e = std::fabs(double(y16[i]) - want_y[i]);
      mx = std::max(mx, e);
      ss += want_y[i] * want_y[i];
      sa += e;
      sr += std::fabs(want_y[i]);
    }
    const double rms = std::sqrt(ss / H);
    std::printf("     BF16 route down + residual: max |y - ref| / rms = %.3g, mean rel = %.3g\n", mx / rms, sa / sr);
    expect(mx <= 1e-3 * rms && sa / sr <= 1e-5,
           "BF16 route: down projection + residual within the north-star tolerance of the oracle");
    auto bad = R::bind_mlp_plan(model, session, 1, s, io, R::MlpRoute::Bf16);
    expect(!bad, "BF16 route rejects repacked (non-0x020D) weights");
  }
  {
    // decode token captured once, replayed per token
    auto plan = unwrap(R::bind_mlp_plan(model, session, 1, s, io), "bind");
    auto graph = unwrap(R::DecodeMlpGraph::capture(plan), "capture");
    bool all = true;
    for (int t = 0; t < 4; ++t) {
      const auto x = uniform(H, 31 + t, 2.f);
      put(h_mid, x, s);
      must(R::execute_decode_mlp(plan), "eager");
      const auto eager = get<float>(next_h, H, s);
      must(zero(next_h.b, s), "zero");
      must(graph.launch(), "replay");
      must(graph.complete_unit(), "complete_unit");
      all = all && same_bits(get<float>(next_h, H, s), eager);
    }
    expect(all, "captured decode token equals the eager submission bitwise on 4 replays with new inputs");
    // capture is rejected by the public synchronous entry point
    {
      auto cap = unwrap(Graph::begin(s), "begin");
      auto r = R::execute_decode_mlp(plan);
      (void)cap.finish();
      expect(!r, "execute_decode_mlp rejects a capturing stream");
    }
    // a nonfinite activation: reported at completion, session poisoned
    auto x = uniform(H, 41, 2.f);
    x[77] = std::nanf("");
    put(h_mid, x, s);
    must(graph.launch(), "replay");
    auto r = graph.complete_unit();
    expect(!r && r.error().operation == "q8.producer", "nonfinite producer reported by complete_unit");
    expect(session.state().is_poisoned() && !graph.launch() && !R::execute_decode_mlp(plan),
           "session poisoned: later submissions rejected");
  }
  {
    // prefill chunks on a fresh session
    auto s2 = unwrap(R::Session::create(s, 64), "session");
    auto engine = unwrap(PrefillEngine::create(s, 128), "PrefillEngine::create");
    const std::uint32_t m = 48;
    put(h_mid, uniform(std::size_t(m) * H, 51, 2.f), s);
    auto plan = unwrap(R::bind_mlp_plan(model, s2, 1, s, io), "bind");
    must(R::execute_prefill_mlp(plan, engine, h_mid.as<float>(), next_h.as<float>(), m, 0), "prefill Q8");
    const auto y = get<float>(next_h, std::size_t(m) * H, s);
    bool submitted = false;
    must(q4k_q8_mlp(plan.gate, plan.up, plan.down, h_mid.as<float>(), plan.gamma, plan.eps, ref.as<float>(), m,
                    {ws.b.as_bytes(), std::size_t(ws.b.bytes())}, s, submitted),
         "direct");
    expect(same_bits(y, get<float>(ref, std::size_t(m) * H, s)),
           "prefill Q8 route (48 tokens, layer 1) equals a direct q4k_q8_mlp bitwise");
    auto p16 = unwrap(R::bind_mlp_plan(model, s2, 0, s, io, R::MlpRoute::Bf16), "bind BF16");
    must(R::execute_prefill_mlp(p16, engine, h_mid.as<float>(), next_h.as<float>(), m, 0), "prefill BF16");
    const auto y16 = get<float>(next_h, std::size_t(m) * H, s);
    must(engine.mlp(p16.gate, p16.up, p16.down, h_mid.as<float>(), p16.gamma, p16.eps, ref.as<float>(), m, 0),
         "engine.mlp");
    expect(same_bits(y16, get<float>(ref, std::size_t(m) * H, s)),
           "prefill BF16 route equals PrefillEngine::mlp bitwise");
    auto over = R::execute_prefill_mlp(plan, engine, h_mid.as<float>(), next_h.as<float>(), 65, 0);
    expect(!over, "prefill chunk beyond the session workspace rejected");
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc > 1 && std::strcmp(argv[1], "--list") == 0) {
    std::printf("runtime_mlp\n");
    return 0;
  }
  auto stream = Stream::create();
  if (!stream) { std::printf("FAIL stream\n"); return 2; }
  std::printf("== runtime_mlp\n");
  run(*stream);
  if (!stream->sync()) return 2;
  std::printf("%d failure(s)\n", g_failures);
  return g_failures == 0 ? 0 : 1;
}
