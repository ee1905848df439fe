// HBM-streaming GEMV for M = 1..8 tokens over 8-row x K256 weight tiles
// (Q4_K layouts 0x020D / 0x0240, Q6_K layout 0x0241) against Q8 activations.
//
// Work mapping (one wave64 per 8-row strip and K-chunk of 8 super-blocks):
//   lane = (kq, g) with kq = lane >> 3 (super-block within the chunk) and
//   g = lane & 7 (K32 group). Each lane loads 16 B of codes per row for its
//   (super-block, group) -- eight consecutive lanes read one contiguous 128 B
//   tile row, so every 16 B load instruction of the wave touches 8 fully used
//   128 B lines -- and reuses its 32 activation bytes per token across the
//   strip's 8 rows. Integer K32 dots use v_dot4_i32_i8 and reset per group
//   (|dot| <= 60960); the FP32 affine a*(ds*dot - dm*sum) per (row, token,
//   group) follows cuda/q4k_q8.cu:97. Per-lane partials are reduced with a
//   transpose-reduce butterfly, then across the waves that split K.
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

// ---- Q4_K unpack: 16 code bytes of one K32 group -> 8 int8x4 vectors in
// logical order (vector j holds codes 4j..4j+3). -----------------------------
template <uint16_t Layout>
__device__ __forceinline__ void q4_unpack(const uint32_t w[4], uint32_t v[8]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = w[t] & 0x0f0f0f0fu;
    const uint32_t hi = (w[t] >> 4) & 0x0f0f0f0fu;
    if constexpr (Layout == QW38_LAYOUT_Q4K_WAVE64) {
      v[2 * t] = lo;      // codes 8t..8t+3
      v[2 * t + 1] = hi;  // codes 8t+4..8t+7
    } else {
      // sequential pairs: lo = c0,c2,c4,c6 and hi = c1,c3,c5,c7
      v[2 * t] = perm(hi, lo, 0x05010400u);
      v[2 * t + 1] = perm(hi, lo, 0x07030602u);
    }
  }
}

__device__ __forceinline__ int dot32(const uint32_t v[8], const uint32_t z[8]) {
  int d = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) d = dot4(v[i], z[i], d);
  return d;
}

// Q6_K: low nibbles (16 B, wave64 nibble order) + high pairs (8 B) -> 8 vectors
// of unsigned 6-bit codes 0..63.
__device__ __forceinline__ void q6_unpack(const uint32_t w[4], const uint32_t h[2],
                                          uint32_t v[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t nib = (j & 1) ? (w[j >> 1] >> 4) & 0x0f0f0f0fu : w[j >> 1] & 0x0f0f0f0fu;
    const uint32_t hh = (h[j >> 2] >> (2 * (j & 3))) & 0x03030303u;
    v[j] = nib | (hh << 4);
  }
}

template <bool Fast>
__device__ __forceinline__ void load16(const uint8_t* p, uint32_t w[4]) {
  if constexpr (Fast) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = q[i];
  }
}

// 16 B of Q4_K metadata: fp16 d, fp16 dmin, 12 packed bytes. The slow path
// tolerates the reference's 2-byte alignment of the scales span.
template <bool Fast>
__device__ __forceinline__ void load_meta(const uint8_t* p, uint32_t m[4]) {
  if constexpr (Fast) {
    load16<true>(p, m);
  } else {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) m[i] = uint32_t(q[2 * i]) | (uint32_t(q[2 * i + 1]) << 16);
  }
}

template <bool Fast>
__device__ __forceinline__ void load_act(const int8_t* p, uint32_t z[8]) {
  if constexpr (Fast) {
    const uint4 a = reinterpret_cast<const uint4*>(p)[0];
    const uint4 b = reinterpret_cast<const uint4*>(p)[1];
    z[0] = a.x; z[1] = a.y; z[2] = a.z; z[3] = a.w;
    z[4] = b.x; z[5] = b.y; z[6] = b.z; z[7] = b.w;
  } else {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = q[i];
  }
}

// Transpose-reduce of acc[8] (rows) over the 64 lanes: after the xor-32/16/8
// exchanges lane L owns row (L >> 3); xor-4/2/1 then sums the 8 groups. Every
// lane of a row-octet ends with that row's total.
__device__ __forceinline__ float reduce_rows(const float acc[8]) {
  const uint32_t lane = threadIdx.x & 63u;
  const bool b5 = lane & 32u, b4 = lane & 16u, b3 = lane & 8u;
  float k1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float send = b5 ? acc[i] : acc[4 + i];
    const float keep = b5 ? acc[4 + i] : acc[i];
    k1[i] = keep + __shfl_xor(send, 32);
  }
  float k2[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float send = b4 ? k1[i] : k1[2 + i];
    const float keep = b4 ? k1[2 + i] : k1[i];
    k2[i] = keep + __shfl_xor(send, 16);
  }
  float v = (b3 ? k2[1] : k2[0]) + __shfl_xor(b3 ? k2[0] : k2[1], 8);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 1);
  return v;
}

// Block = 4 waves; WS waves split the K chunks of one strip; 4/WS strips per block.
// At least two waves per SIMD (at most 256 registers): Q6_K at M=8 would take
// 266 and run one wave per SIMD (62.6 us at config 3 against 52.6 us here).
template <uint16_t Layout, int MT, bool Fast, int WS>
__global__ __launch_bounds__(256, 2) void gemv_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n,
    uint32_t strips, uint32_t kbs, const int8_t* __restrict__ xc,
    const float* __restrict__ xa, const int32_t* __restrict__ xs, uint32_t pk,
    float* __restrict__ out, const float* __restrict__ residual) {
  constexpr int SPB = 4 / WS;
  __shared__ float red[WS > 1 ? 4 * MT * 8 : 1];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t strip = blockIdx.x * SPB + wave / WS;
  const uint32_t ks = wave % WS;
  const uint32_t kq = lane >> 3, g = lane & 7u;
  const uint32_t groups = pk / 32;
  const bool live = strip < strips;

  float acc[MT][8];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[t][r] = 0.f;

  constexpr bool kQ6 = Layout == QW38_LAYOUT_Q6K_WAVE64;
  constexpr uint32_t kRowBytes = kQ6 ? kQ6CodeBytes : kQ4CodeBytes;
  const uint8_t* cstrip = codes + size_t(strip) * kbs * 8 * kRowBytes;
  const uint8_t* mstrip = meta + size_t(strip) * kbs * 8 * 16;
  // Q6_K fp16 d array follows the 16-byte scale rows of all tiles.
  const uint8_t* dstrip = meta + size_t(strips) * 8 * kbs * 16 + size_t(strip) * kbs * 8 * 2;

  if (live) {
    for (uint32_t c = ks; c * 8 < kbs; c += WS) {
      const uint32_t kb = c * 8 + kq;
      if (kb >= kbs) continue;
      uint32_t z[MT][8];
      float a[MT], fs[MT];
      int zs0[MT], zs1[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const size_t gi = size_t(t) * groups + kb * 8 + g;
        load_act<Fast>(xc + gi * 32, z[t]);
        a[t] = xa[gi];
        fs[t] = float(xs[gi]);
        if constexpr (kQ6) {
          zs0[t] = dot4(0x01010101u, z[t][0], dot4(0x01010101u, z[t][1],
                   dot4(0x01010101u, z[t][2], dot4(0x01010101u, z[t][3], 0))));
          zs1[t] = dot4(0x01010101u, z[t][4], dot4(0x01010101u, z[t][5],
                   dot4(0x01010101u, z[t][6], dot4(0x01010101u, z[t][7], 0))));
        }
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        if constexpr (!kQ6) {
          uint32_t w[4], mt[4], v[8];
          load16<Fast>(cstrip + size_t(kb) * 1024 + r * 128 + g * 16, w);
          load_meta<Fast>(mstrip + size_t(kb) * 128 + r * 16, mt);
          float s, m;
          q4_scale_min_lane(mt[1], mt[2], mt[3], g, s, m);
          const float ds = f16_to_f32(mt[0] & 0xffffu) * s;
          const float dm = f16_to_f32(mt[0] >> 16) * m;
          q4_unpack<Layout>(w, v);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const int dot = dot32(v, z[t]);
            acc[t][r] = fmaf(a[t], fmaf(ds, float(dot), -(dm * fs[t])), acc[t][r]);
          }
        } else {
          uint32_t w[4], h[2], v[8];
          const uint8_t* tile = cstrip + size_t(kb) * kQ6TileBytes;
          load16<true>(tile + q6_chunk(r, g) * 16, w);
          const uint2 hv = *reinterpret_cast<const uint2*>(tile + kQ6HiPlane + q6_chunk(r, g) * 8);
          h[0] = hv.x; h[1] = hv.y;
          const uint16_t scw = *reinterpret_cast<const uint16_t*>(
              mstrip + size_t(kb) * 128 + r * 16 + g * 2);
          const int sc0 = int(int8_t(scw & 0xffu)), sc1 = int(int8_t(scw >> 8));
          const float d = f16_to_f32(
              *reinterpret_cast<const uint16_t*>(dstrip + (size_t(kb) * 8 + r) * 2));
          q6_unpack(w, h, v);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            int d0 = 0, d1 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) d0 = dot4(v[i], z[t][i], d0);
#pragma unroll
            for (int i = 4; i < 8; ++i) d1 = dot4(v[i], z[t][i], d1);
            const int I = sc0 * (d0 - 32 * zs0[t]) + sc1 * (d1 - 32 * zs1[t]);
            acc[t][r] = fmaf(a[t], d * float(I), acc[t][r]);
          }
        }
      }
    }
  }

  const uint32_t row = strip * 8 + (lane >> 3);
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const float total = reduce_rows(acc[t]);
    if constexpr (WS == 1) {
      if (live && (lane & 7u) == 0 && row < n) {
        const size_t i = size_t(t) * n + row;
        out[i] = total + (residual ? residual[i] : 0.f);
      }
    } else {
      if ((lane & 7u) == 0) red[(wave * MT + t) * 8 + (lane >> 3)] = total;
    }
  }
  if constexpr (WS > 1) {
    __syncthreads();
    if (live && ks == 0 && (lane & 7u) == 0 && row < n) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        float total = 0.f;
#pragma unroll
        for (int j = 0; j < WS; ++j) total += red[((wave + j) * MT + t) * 8 + (lane >> 3)];
        const size_t i = size_t(t) * n + row;
        out[i] = total + (residual ? residual[i] : 0.f);
      }
    }
  }
}

// Per-(token, row, group) int32 dots through the same unpack/dot routines.
template <uint16_t Layout>
__global__ void group_dots_kernel(const uint8_t* __restrict__ codes,
                                  const uint8_t* __restrict__ meta, uint32_t n,
                                  uint32_t strips, uint32_t kbs, const int8_t* __restrict__ xc,
                                  uint32_t pk, uint32_t m, int32_t* __restrict__ dots) {
  const uint32_t groups = pk / 32;
  const uint64_t idx = uint64_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= uint64_t(m) * n * groups) return;
  const uint32_t g_all = uint32_t(idx % groups);
  const uint32_t r = uint32_t((idx / groups) % n);
  const uint32_t t = uint32_t(idx / (uint64_t(groups) * n));
  const uint32_t kb = g_all / 8, g = g_all % 8;
  const uint64_t tr = (uint64_t(r / 8) * kbs + kb) * 8 + r % 8;
  uint32_t z[8], v[8];
  load_act<false>(xc + size_t(t) * pk + size_t(g_all) * 32, z);
  if constexpr (Layout != QW38_LAYOUT_Q6K_WAVE64) {
    uint32_t w[4];
    load16<false>(codes + q4k_code_word(Layout, r, kb, g, kbs, strips), w);
    q4_unpack<Layout>(w, v);
    dots[idx] = dot32(v, z);
  } else {
    uint32_t w[4], h[2];
    const uint8_t* tile = codes + (tr - r % 8) * kQ6CodeBytes;
    load16<false>(tile + q6_chunk(r % 8, g) * 16, w);
    h[0] = *reinterpret_cast<const uint32_t*>(tile + kQ6HiPlane + q6_chunk(r % 8, g) * 8);
    h[1] = *reinterpret_cast<const uint32_t*>(tile + kQ6HiPlane + q6_chunk(r % 8, g) * 8 + 4);
    q6_unpack(w, h, v);
    const uint16_t scw = *reinterpret_cast<const uint16_t*>(meta + tr * 16 + g * 2);
    const int sc0 = int(int8_t(scw & 0xffu)), sc1 = int(int8_t(scw >> 8));
    int d0 = 0, d1 = 0, s0 = 0, s1 = 0;
    for (int i = 0; i < 4; ++i) {
      d0 = dot4(v[i], z[i], d0);
      s0 = dot4(0x01010101u, z[i], s0);
    }
    for (int i = 4; i < 8; ++i) {
      d1 = dot4(v[i], z[i], d1);
      s1 = dot4(0x01010101u, z[i], s1);
    }
    dots[idx] = sc0 * (d0 - 32 * s0) + sc1 * (d1 - 32 * s1);
  }
  (void)strips;
}

template <uint16_t Layout, int MT, bool Fast>
hipError_t gemv_ws(const WeightView& w, const Q8View& x, float* out, const float* residual,
                   hipStream_t s) {
  const uint32_t strips = w.pn / 8, kbs = w.pk / 256;
  const uint32_t chunks = (kbs + 7) / 8;
  // Enough waves to cover the chip (256 CUs) several times over; split K
  // across up to 4 waves of a block when the strip count alone is too low.
  int ws = 1;
  if (strips < 4096 && chunks >= 2) ws = 2;
  if (strips < 2048 && chunks >= 4) ws = 4;
  // Tuning override for measurement sweeps (1, 2 or 4 waves per strip).
  static const int ws_env = [] {
    const char* e = std::getenv("QW38_GEMV_WS");
    return e ? std::atoi(e) : 0;
  }();
  if (ws_env == 1 || ws_env == 2 || ws_env == 4) ws = ws_env;
#define QW38_GEMV_LAUNCH(WSV)                                                               \
  hipLaunchKernelGGL((gemv_kernel<Layout, MT, Fast, WSV>),                                 \
                     dim3((strips + (4 / WSV) - 1) / (4 / WSV)), dim3(256), 0, s, w.codes, \
                     w.scales, w.n, strips, kbs, x.codes, x.scales, x.sums, x.pk, out,     \
                     residual)
  if (ws == 4) QW38_GEMV_LAUNCH(4);
  else if (ws == 2) QW38_GEMV_LAUNCH(2);
  else QW38_GEMV_LAUNCH(1);
#undef QW38_GEMV_LAUNCH
  return hipGetLastError();
}

template <uint16_t Layout, bool Fast>
hipError_t gemv_m(const WeightView& w, const Q8View& x, float* out, const float* residual,
                  hipStream_t s) {
  switch (x.m) {
    case 1: return gemv_ws<Layout, 1, Fast>(w, x, out, residual, s);
    case 2: return gemv_ws<Layout, 2, Fast>(w, x, out, residual, s);
    case 3: return gemv_ws<Layout, 3, Fast>(w, x, out, residual, s);
    case 4: return gemv_ws<Layout, 4, Fast>(w, x, out, residual, s);
    case 5: return gemv_ws<Layout, 5, Fast>(w, x, out, residual, s);
    case 6: return gemv_ws<Layout, 6, Fast>(w, x, out, residual, s);
    case 7: return gemv_ws<Layout, 7, Fast>(w, x, out, residual, s);
    case 8: return gemv_ws<Layout, 8, Fast>(w, x, out, residual, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gemv(const WeightView& w, const Q8View& x, float* out, const float* residual,
                       hipStream_t s) {
  // Tuning knobs for measurement sweeps: QW38_GEMV_STREAM=0 disables the
  // linear-streaming kernel; QW38_GEMV_STREAM_WS / _BLOCKS override its shape.
  static const int env_stream = [] {
    const char* e = std::getenv("QW38_GEMV_STREAM");
    return e ? std::atoi(e) : 1;
  }();
  static const int env_ws = [] {
    const char* e = std::getenv("QW38_GEMV_STREAM_WS");
    return e ? std::atoi(e) : 0;
  }();
  static const int env_blocks = [] {
    const char* e = std::getenv("QW38_GEMV_STREAM_BLOCKS");
    return e ? std::atoi(e) : 0;
  }();
  {
    const hipError_t e = launch_q4k_mfma_decode(w, x, out, residual, s);
    if (e != hipErrorNotSupported) return e;
  }
  if (env_stream) {
    const hipError_t e = launch_gemv_stream(w, x, out, residual, s, env_ws, uint32_t(env_blocks));
    if (e != hipErrorNotSupported) return e;
  }
  const bool fast = (reinterpret_cast<uintptr_t>(w.codes) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(w.scales) % 16 == 0) &&
                    (reinterpret_cast<uintptr_t>(x.codes) % 16 == 0);
  switch (w.layout) {
    case QW38_LAYOUT_Q4K_CANDIDATE_V2:
      return fast ? gemv_m<QW38_LAYOUT_Q4K_CANDIDATE_V2, true>(w, x, out, residual, s)
                  : gemv_m<QW38_LAYOUT_Q4K_CANDIDATE_V2, false>(w, x, out, residual, s);
    case QW38_LAYOUT_Q4K_WAVE64:
      return launch_gemv_w64(w, x, out, residual, s);
    case QW38_LAYOUT_Q6K_WAVE64: {
      hipError_t e = launch_q6k_mfma_decode(w, x, out, residual, s);
      if (e != hipErrorNotSupported) return e;
      e = launch_q6k_stream(w, x, out, residual, s);
      if (e != hipErrorNotSupported) return e;
    }
      // Q6_K layout requires 16-byte aligned codes (validated by the caller).
      return (reinterpret_cast<uintptr_t>(x.codes) % 16 == 0)
                 ? gemv_m<QW38_LAYOUT_Q6K_WAVE64, true>(w, x, out, residual, s)
                 : gemv_m<QW38_LAYOUT_Q6K_WAVE64, false>(w, x, out, residual, s);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_group_dots(const WeightView& w, const Q8View& x, int32_t* dots,
                             hipStream_t s) {
  const uint32_t strips = w.pn / 8, kbs = w.pk / 256;
  const uint64_t total = uint64_t(x.m) * w.n * (w.pk / 32);
  const dim3 grid(uint32_t((total + 255) / 256));
  switch (w.layout) {
    case QW38_LAYOUT_Q4K_CANDIDATE_V2:
      hipLaunchKernelGGL(group_dots_kernel<QW38_LAYOUT_Q4K_CANDIDATE_V2>, grid, dim3(256), 0, s,
                         w.codes, w.scales, w.n, strips, kbs, x.codes, x.pk, x.m, dots);
      break;
    case QW38_LAYOUT_Q4K_WAVE64:
      hipLaunchKernelGGL(group_dots_kernel<QW38_LAYOUT_Q4K_WAVE64>, grid, dim3(256), 0, s,
                         w.codes, w.scales, w.n, strips, kbs, x.codes, x.pk, x.m, dots);
      break;
    case QW38_LAYOUT_Q6K_WAVE64:
      hipLaunchKernelGGL(group_dots_kernel<QW38_LAYOUT_Q6K_WAVE64>, grid, dim3(256), 0, s,
                         w.codes, w.scales, w.n, strips, kbs, x.codes, x.pk, x.m, dots);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace qw38hip
