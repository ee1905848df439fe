// Decode GEMV (M = 1..8 tokens) over the wave64 plane layout 0x0240.
//
// Layout: per 8-row strip and chunk of nk <= 8 super-blocks, the codes form
// eight planes (one per K32 group) of nk*128 B whose 16-byte entries are in
// lane order (kb%8)*8 + row%8; the metadata is the 0x020D tile-row array,
// which within a chunk is in the same lane order. Lane l = 8*kq + r of a wave
// therefore owns the whole super-block (row r, kb = 8c + kq): eight 16 B code
// loads and one 16 B metadata load per chunk, each wave instruction reading
// one contiguous plane (1 KB for a full chunk). Nothing is exchanged between
// lanes until the final row reduction, and each lane decodes its super-block
// metadata once for all eight groups.
//
// Arithmetic per (row, token, super-block), exact int32 K32 dots from
// v_dot4_i32_i8, FP32 affine reassociated from the reference's
// sum_g a_g (d s_g dot_g - dmin m_g sum_g) (cuda/q4k_q8.cu:97):
//   X = sum_g a_g * float(s_g * dot_g),  Y = sum_g (a_g sum_g) * m_g,
//   acc += d * X - dmin * Y.
// The Q8 activations are staged once per block in LDS (codes and (a, a*sum)).
// Row totals: butterfly over the 8 lanes of a row (xor 8, 16, 32), then over
// the WS waves that split the strip's chunks, in a fixed order.
#include <cstdlib>

#include "common.hpp"

namespace qw38hip {
namespace {

template <int MT, bool FastAct, bool ActLds, int WS>
__global__ __launch_bounds__(256) void gemv_w64_kernel(
    const uint8_t* __restrict__ codes, const uint8_t* __restrict__ meta, uint32_t n,
    uint32_t strips, uint32_t kbs, const int8_t* __restrict__ xc,
    const float* __restrict__ xa, const int32_t* __restrict__ xs, uint32_t pk,
    float* __restrict__ out, const float* __restrict__ residual) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int SPB = 4 / WS;
  const uint32_t groups = pk / 32;
  int8_t* sz = reinterpret_cast<int8_t*>(smem);
  float2* sau = reinterpret_cast<float2*>(smem + MT * pk);
  float* red = reinterpret_cast<float*>(ActLds ? smem + MT * pk + MT * groups * 8 : smem);

  // Activations too large for LDS (long K at larger M) are read through the
  // caches instead; the arithmetic is identical.
  if constexpr (ActLds) {
    if constexpr (FastAct) {
      const uint4* src = reinterpret_cast<const uint4*>(xc);
      uint4* dst = reinterpret_cast<uint4*>(sz);
      for (uint32_t i = threadIdx.x; i < MT * pk / 16; i += 256) dst[i] = src[i];
    } else {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(xc);
      uint32_t* dst = reinterpret_cast<uint32_t*>(sz);
      for (uint32_t i = threadIdx.x; i < MT * pk / 4; i += 256) dst[i] = src[i];
    }
    for (uint32_t i = threadIdx.x; i < MT * groups; i += 256) {
      const float a = xa[i];
      sau[i] = make_float2(a, a * float(xs[i]));
    }
    __syncthreads();
  }

  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t kq = lane >> 3, r = lane & 7u;
  const uint32_t ks = wave % WS;
  const uint32_t strip = blockIdx.x * SPB + wave / WS;
  const bool live = strip < strips;
  const uint32_t chunks = (kbs + 7) / 8;
  const uint32_t c0 = uint32_t(uint64_t(chunks) * ks / WS);
  const uint32_t c1 = uint32_t(uint64_t(chunks) * (ks + 1) / WS);

  float acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = 0.f;

  if (live) {
    for (uint32_t c = c0; c < c1; ++c) {
      const uint32_t nk = min(8u, kbs - 8 * c);
      const uint32_t kb = 8 * c + kq;
      if (kq < nk) {
        // chunk-major: chunk c of all strips, then this strip's nk super-blocks
        const uint8_t* cb = codes + size_t(strips) * 8192 * c + size_t(strip) * nk * 1024 + lane * 16;
        const uint8_t* mb = meta + size_t(strips) * 1024 * c + size_t(strip) * nk * 128 + lane * 16;
        const uint32_t plane = nk * 128;
        uint4 w[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) w[g] = *reinterpret_cast<const uint4*>(cb + g * plane);
        const uint4 mt = *reinterpret_cast<const uint4*>(mb);
        const float d = f16_to_f32(mt.x & 0xffffu), dmin = f16_to_f32(mt.x >> 16);
        // 6-bit scales/mins of the 8 groups (get_scale_min_k4 with constant g)
        uint32_t sc[8];
        float mf[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          uint32_t s, m;
          q4k_scale_min(mt.y, mt.z, mt.w, g, s, m);
          sc[g] = s;
          mf[g] = float(m);
        }
        float X[MT], Y[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) X[t] = Y[t] = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const uint32_t ww[4] = {w[g].x, w[g].y, w[g].z, w[g].w};
          uint32_t v[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            v[2 * q] = ww[q] & 0x0f0f0f0fu;
            v[2 * q + 1] = (ww[q] >> 4) & 0x0f0f0f0fu;
          }
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const uint32_t gi = t * groups + kb * 8 + g;
            uint4 za, zb;
            float2 au;
            if constexpr (ActLds) {
              const uint4* zp = reinterpret_cast<const uint4*>(sz + size_t(gi) * 32);
              za = zp[0];
              zb = zp[1];
              au = sau[gi];
            } else {
              if constexpr (FastAct) {
                const uint4* zp = reinterpret_cast<const uint4*>(xc + size_t(gi) * 32);
                za = zp[0];
                zb = zp[1];
              } else {
                const uint32_t* zp = reinterpret_cast<const uint32_t*>(xc + size_t(gi) * 32);
                za = make_uint4(zp[0], zp[1], zp[2], zp[3]);
                zb = make_uint4(zp[4], zp[5], zp[6], zp[7]);
              }
              const float a = xa[gi];
              au = make_float2(a, a * float(xs[gi]));
            }
            int dot = 0;
            dot = dot4(v[0], za.x, dot);
            dot = dot4(v[1], za.y, dot);
            dot = dot4(v[2], za.z, dot);
            dot = dot4(v[3], za.w, dot);
            dot = dot4(v[4], zb.x, dot);
            dot = dot4(v[5], zb.y, dot);
            dot = dot4(v[6], zb.z, dot);
            dot = dot4(v[7], zb.w, dot);
            X[t] = fmaf(au.x, float(__mul24(dot, int(sc[g]))), X[t]);
            Y[t] = fmaf(au.y, mf[g], Y[t]);
          }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = fmaf(-dmin, Y[t], fmaf(d, X[t], acc[t]));
      }
    }
  }
  // a row's super-block partials live in lanes r, r+8, ..., r+56
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    acc[t] += __shfl_xor(acc[t], 8);
    acc[t] += __shfl_xor(acc[t], 16);
    acc[t] += __shfl_xor(acc[t], 32);
  }
  const uint32_t row = strip * 8 + r;
  if constexpr (WS == 1) {
    if (live && kq == 0 && row < n) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const size_t i = size_t(t) * n + row;
        out[i] = acc[t] + (residual ? residual[i] : 0.f);
      }
    }
  } else {
    if (kq == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) red[(wave * MT + t) * 8 + r] = acc[t];
    }
    __syncthreads();
    if (live && ks == 0 && kq == 0 && row < n) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        float total = 0.f;
#pragma unroll
        for (int q = 0; q < WS; ++q) total += red[((wave + q) * MT + t) * 8 + r];
        const size_t i = size_t(t) * n + row;
        out[i] = total + (residual ? residual[i] : 0.f);
      }
    }
  }
}

constexpr size_t kMaxActLds = 56 * 1024;

template <int MT, bool FastAct, bool ActLds>
hipError_t w64_ws(const WeightView& w, const Q8View& x, float* out, const float* residual,
                  hipStream_t s, int ws) {
  const uint32_t strips = w.pn / 8, kbs = w.pk / 256;
  const size_t lds = ActLds ? size_t(MT) * w.pk + size_t(MT) * (w.pk / 32) * 8 + 4 * MT * 8 * 4
                            : size_t(4 * MT * 8 * 4);
#define QW38_W64_LAUNCH(WSV)                                                              \
  hipLaunchKernelGGL((gemv_w64_kernel<MT, FastAct, ActLds, WSV>),                                 \
                     dim3((strips + (4 / WSV) - 1) / (4 / WSV)), dim3(256), lds, s, w.codes, \
                     w.scales, w.n, strips, kbs, x.codes, x.scales, x.sums, x.pk, out, residual)
  if (ws == 4) QW38_W64_LAUNCH(4);
  else if (ws == 2) QW38_W64_LAUNCH(2);
  else QW38_W64_LAUNCH(1);
#undef QW38_W64_LAUNCH
  return hipGetLastError();
}

template <int MT, bool FastAct>
hipError_t w64_lds(const WeightView& w, const Q8View& x, float* out, const float* residual,
                   hipStream_t s, int ws) {
  const size_t need = size_t(MT) * w.pk * 5 / 4 + 4 * MT * 8 * 4;
  return need <= kMaxActLds ? w64_ws<MT, FastAct, true>(w, x, out, residual, s, ws)
                            : w64_ws<MT, FastAct, false>(w, x, out, residual, s, ws);
}

template <bool FastAct>
hipError_t w64_m(const WeightView& w, const Q8View& x, float* out, const float* residual,
                 hipStream_t s, int ws) {
  switch (x.m) {
    case 1: return w64_lds<1, FastAct>(w, x, out, residual, s, ws);
    case 2: return w64_lds<2, FastAct>(w, x, out, residual, s, ws);
    case 3: return w64_lds<3, FastAct>(w, x, out, residual, s, ws);
    case 4: return w64_lds<4, FastAct>(w, x, out, residual, s, ws);
    case 5: return w64_lds<5, FastAct>(w, x, out, residual, s, ws);
    case 6: return w64_lds<6, FastAct>(w, x, out, residual, s, ws);
    case 7: return w64_lds<7, FastAct>(w, x, out, residual, s, ws);
    case 8: return w64_lds<8, FastAct>(w, x, out, residual, s, ws);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gemv_w64(const WeightView& w, const Q8View& x, float* out,
                           const float* residual, hipStream_t s) {
  const uint32_t strips = w.pn / 8, chunks = (w.pk / 256 + 7) / 8;
  int ws = 1;
  if (strips < 2048 && chunks >= 2) ws = 2;
  if (strips < 1024 && chunks >= 4) ws = 4;
  static const int env_ws = [] {
    const char* e = std::getenv("QW38_GEMV_W64_WS");
    return e ? std::atoi(e) : 0;
  }();
  if (env_ws == 1 || env_ws == 2 || env_ws == 4) ws = env_ws;
  const bool fast_act = reinterpret_cast<uintptr_t>(x.codes) % 16 == 0;
  return fast_act ? w64_m<true>(w, x, out, residual, s, ws)
                  : w64_m<false>(w, x, out, residual, s, ws);
}

}  // namespace qw38hip
