// On-device Q4_K / Q6_K fitting of FP32 rows into GGML-order super-blocks
// (then repacked by repack.hip). Follows the reference's production fitter
// (src/compiler/quantization/q4k.cpp:186-278, a port of llama.cpp
// quantize_row_q4_K_ref, third_party/llama.cpp-q4k/reference.hpp:93-252) with
// the same FP32 operation order, no contraction and IEEE div/sqrt, so the
// output bytes equal the CPU fitter's. Q6_K follows llama.cpp
// quantize_row_q6_K_ref / make_qx_quants (not vendored in the reference).
//
// Mapping: one lane per K32 group (Q4_K) or per 16-value sub-block (Q6_K);
// the lanes of one 256-value super-block combine their scales by shuffles.
#include "common.hpp"

namespace qw38hip {
namespace {

__device__ __forceinline__ int nearest_int(float f) {
  const float v = f + 12582912.f;
  return int(__float_as_uint(v) & 0x007fffffu) - 0x00400000;
}

// IEEE round-to-nearest-even FP32 -> FP16 bits (NaN -> 0x7e00).
__device__ __forceinline__ uint16_t to_fp16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint16_t sign = uint16_t((u >> 16) & 0x8000u);
  const uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return sign | 0x7e00u;
  if (au >= 0x477ff000u) return sign | 0x7c00u;
  if (au < 0x38800000u) {
    const double q = double(__uint_as_float(au)) * 16777216.0;
    return sign | uint16_t(rint(q));
  }
  const uint32_t exp = (au >> 23) - 112u, mant = au & 0x7fffffu;
  uint32_t h = (exp << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return sign | uint16_t(h);
}

__device__ float fit_qkx2(const float* x, const float* w, uint8_t* L, float* the_min,
                          uint8_t* Laux) {
  const int n = 32, nmax = 15, nstep = 20;
  const float rmin = -1.f, rdelta = 0.1f;
  float mn = x[0], mx = x[0];
  float sum_w = w[0];
  float sum_x = sum_w * x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < mn) mn = x[i];
    if (x[i] > mx) mx = x[i];
    const float wi = w[i];
    sum_w += wi;
    sum_x += wi * x[i];
  }
  if (mn > 0) mn = 0;
  if (mx == mn) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    *the_min = -mn;
    return 0.f;
  }
  float iscale = nmax / (mx - mn);
  float scale = 1 / iscale;
  float best = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * (x[i] - mn));
    L[i] = uint8_t(l < 0 ? 0 : l > nmax ? nmax : l);
    float diff = scale * L[i] + mn - x[i];
    diff = diff * diff;
    best += w[i] * diff;
  }
  for (int is = 0; is <= nstep; ++is) {
    iscale = (rmin + rdelta * is + nmax) / (mx - mn);
    float sl = 0, sl2 = 0, sxl = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * (x[i] - mn));
      l = l < 0 ? 0 : l > nmax ? nmax : l;
      Laux[i] = uint8_t(l);
      const float wi = w[i];
      sl += wi * l;
      sl2 += wi * l * l;
      sxl += wi * l * x[i];
    }
    const float D = sum_w * sl2 - sl * sl;
    if (D > 0) {
      float ts = (sum_w * sxl - sum_x * sl) / D;
      float tm = (sl2 * sum_x - sl * sxl) / D;
      if (tm > 0) {
        tm = 0;
        ts = sxl / sl2;
      }
      float cur = 0;
      for (int i = 0; i < n; ++i) {
        float diff = ts * Laux[i] + tm - x[i];
        diff = diff * diff;
        cur += w[i] * diff;
      }
      if (cur < best) {
        for (int i = 0; i < n; ++i) L[i] = Laux[i];
        best = cur;
        scale = ts;
        mn = tm;
      }
    }
  }
  *the_min = -mn;
  return scale;
}

// 8 lanes per super-block (lane & 7 = group); 32 super-blocks per 256 threads.
__global__ __launch_bounds__(256) void quantize_q4k_kernel(const float* __restrict__ x,
                                                           uint64_t blocks,
                                                           uint8_t* __restrict__ out,
                                                           int* failure) {
  const uint64_t blk = uint64_t(blockIdx.x) * 32 + (threadIdx.x >> 3);
  const uint32_t j = threadIdx.x & 7u;
  const bool live = blk < blocks;
  float xs[32], w[32];
  uint8_t L[32], aux[32];
  int err = 0;
  float scale = 0.f, minv = 0.f;
  if (live) {
    const float* xj = x + blk * 256 + j * 32;
    for (int i = 0; i < 32; ++i) xs[i] = xj[i];
    float lo = 0, hi = xs[0];
    for (int i = 0; i < 32; ++i) {
      if (!isfinite(xs[i])) err |= 1;
      else if (fabsf(xs[i]) > 1.0e10f) err |= 2;
      lo = fminf(lo, xs[i]);
      hi = fmaxf(hi, xs[i]);
    }
    if (!err && hi != lo && !isfinite(16.f / (hi - lo))) err |= 2;
    if (!err) {
      float sx2 = 0;
      for (int i = 0; i < 32; ++i) sx2 += xs[i] * xs[i];
      const float av = sqrtf(sx2 / 32);
      for (int i = 0; i < 32; ++i) w[i] = av + fabsf(xs[i]);
      scale = fit_qkx2(xs, w, L, &minv, aux);
    }
  }
  // Combine the 8 groups in ascending order, exactly as the sequential loop.
  float max_scale = 0.f, max_min = 0.f;
  int any_err = err;
  for (int g = 0; g < 8; ++g) {
    const float sg = __shfl(scale, (threadIdx.x & ~7u) + g, 64);
    const float mg = __shfl(minv, (threadIdx.x & ~7u) + g, 64);
    any_err |= __shfl(err, (threadIdx.x & ~7u) + g, 64);
    if (sg > max_scale) max_scale = sg;
    if (mg > max_min) max_min = mg;
  }
  if (!live) return;
  if (any_err) {
    if (j == 0) *failure = 1;
    return;
  }
  const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
  const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
  if (!isfinite(inv_scale) || !isfinite(inv_min)) {
    if (j == 0) *failure = 1;
    return;
  }
  uint8_t ls = uint8_t(nearest_int(inv_scale * scale));
  uint8_t lm = uint8_t(nearest_int(inv_min * minv));
  if (ls > 63) ls = 63;
  if (lm > 63) lm = 63;
  const uint16_t d = to_fp16(max_scale / 63.f);
  const uint16_t dmin = to_fp16(max_min / 63.f);
  if ((d & 0x7c00u) == 0x7c00u || (dmin & 0x7c00u) == 0x7c00u) {
    if (j == 0) *failure = 1;
    return;
  }
  // Recompute codes from the compressed 6-bit scale and the rounded FP16 d/dmin.
  const float step = f16_to_f32(d) * float(ls);
  if (step) {
    const float off = f16_to_f32(dmin) * float(lm);
    for (int i = 0; i < 32; ++i) {
      int l = nearest_int((xs[i] + off) / step);
      L[i] = uint8_t(l < 0 ? 0 : l > 15 ? 15 : l);
    }
  }
  // GGML block: d, dmin, 12 packed scale bytes, qs[128].
  uint8_t* y = out + blk * 144;
  const uint32_t base = (threadIdx.x & ~7u);
  // Scale bytes: every lane gathers the 8 (ls, lm) pairs and lane 0 writes them.
  uint32_t sl_all[8], ml_all[8];
  for (int g = 0; g < 8; ++g) {
    sl_all[g] = uint32_t(__shfl(int(ls), base + g, 64));
    ml_all[g] = uint32_t(__shfl(int(lm), base + g, 64));
  }
  if (j == 0) {
    uint8_t p[12] = {0};
    for (int g = 0; g < 8; ++g) {
      if (g < 4) {
        p[g] = uint8_t(sl_all[g]);
        p[g + 4] = uint8_t(ml_all[g]);
      } else {
        p[g + 4] = uint8_t((sl_all[g] & 15) | ((ml_all[g] & 15) << 4));
        p[g - 4] |= uint8_t((sl_all[g] >> 4) << 6);
        p[g] |= uint8_t((ml_all[g] >> 4) << 6);
      }
    }
    y[0] = d & 255;
    y[1] = d >> 8;
    y[2] = dmin & 255;
    y[3] = dmin >> 8;
    for (int i = 0; i < 12; ++i) y[4 + i] = p[i];
  }
  // qs[32c + l] = L[64c + l] | L[64c + 32 + l] << 4: group j holds the low
  // nibbles (j even) or high nibbles (j odd) of chunk c = j / 2.
  const uint32_t c = j / 2;
  const bool high = j & 1u;
  for (int l = 0; l < 32; ++l) {
    const uint32_t mine = L[l];
    const uint32_t other = uint32_t(__shfl(int(mine), threadIdx.x ^ 1u, 64));
    if (!high) y[16 + 32 * c + l] = uint8_t(mine | (other << 4));
  }
}

// ---- Q6_K ------------------------------------------------------------------
__device__ float fit_qx16(const float* x, uint8_t* L) {
  const int n = 16, nmax = 32;
  float max = 0, amax = 0;
  for (int i = 0; i < n; ++i) {
    const float ax = fabsf(x[i]);
    if (ax > amax) {
      amax = ax;
      max = x[i];
    }
  }
  if (amax < 1e-15f) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  float iscale = -nmax / max;
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * x[i]);
    l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
    L[i] = uint8_t(l + nmax);
    const float w = x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  float scale = suml2 ? sumlx / suml2 : 0.0f;
  float best = scale * sumlx;
  for (int is = -9; is <= 9; ++is) {
    if (is == 0) continue;
    iscale = -(nmax + 0.1f * is) / max;
    sumlx = suml2 = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * x[i]);
      l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
      const float w = x[i] * x[i];
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
        L[i] = uint8_t(nmax + l);
      }
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

// 16 lanes per super-block (one 16-value sub-block each); 16 blocks per 256 threads.
__global__ __launch_bounds__(256) void quantize_q6k_kernel(const float* __restrict__ x,
                                                           uint64_t blocks,
                                                           uint8_t* __restrict__ out) {
  const uint64_t blk = uint64_t(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const uint32_t ib = threadIdx.x & 15u;
  const uint32_t base = threadIdx.x & ~15u;
  const bool live = blk < blocks;
  float xs[16];
  uint8_t L[16];
  float s = 0.f;
  if (live) {
    for (int i = 0; i < 16; ++i) xs[i] = x[blk * 256 + ib * 16 + i];
    s = fit_qx16(xs, L);
  }
  float max_scale = 0, max_abs = 0;
  for (int g = 0; g < 16; ++g) {
    const float sg = __shfl(s, base + g, 64);
    const float as = fabsf(sg);
    if (as > max_abs) {
      max_abs = as;
      max_scale = sg;
    }
  }
  if (!live) return;
  uint8_t* y = out + blk * 210;
  int8_t scq = 0;
  uint16_t d = 0;
  if (max_abs < 1e-15f) {
    for (int i = 0; i < 16; ++i) L[i] = 0;
  } else {
    const float iscale = -128.f / max_scale;
    d = to_fp16(1 / iscale);
    const int l = nearest_int(iscale * s);
    scq = int8_t(l < 127 ? l : 127);
    const float dd = f16_to_f32(d) * float(scq);
    if (dd) {
      for (int i = 0; i < 16; ++i) {
        int q = nearest_int(xs[i] / dd);
        q = q < -32 ? -32 : q > 31 ? 31 : q;
        L[i] = uint8_t(q + 32);
      }
    }
  }
  y[192 + ib] = uint8_t(scq);
  if (ib == 0) {
    y[208] = d & 255;
    y[209] = d >> 8;
  }
  // Assemble ql/qh in the lanes of parts 0/1 (ib in 0..3 per half): every lane
  // fetches the codes of the other parts at the same within-part position.
  const uint32_t h = ib / 8, within = ib % 8;  // 8 sub-blocks per half
  const uint32_t p = within / 2, lofs = (within % 2) * 16;
  for (int i = 0; i < 16; ++i) {
    const uint32_t l = lofs + i;
    const uint32_t v0 = uint32_t(__shfl(int(L[i]), base + h * 8 + 0 * 2 + (within % 2), 64));
    const uint32_t v1 = uint32_t(__shfl(int(L[i]), base + h * 8 + 1 * 2 + (within % 2), 64));
    const uint32_t v2 = uint32_t(__shfl(int(L[i]), base + h * 8 + 2 * 2 + (within % 2), 64));
    const uint32_t v3 = uint32_t(__shfl(int(L[i]), base + h * 8 + 3 * 2 + (within % 2), 64));
    if (p == 0) {
      y[64 * h + l] = uint8_t((v0 & 15) | ((v2 & 15) << 4));
      y[64 * h + l + 32] = uint8_t((v1 & 15) | ((v3 & 15) << 4));
      y[128 + 32 * h + l] =
          uint8_t((v0 >> 4) | ((v1 >> 4) << 2) | ((v2 >> 4) << 4) | ((v3 >> 4) << 6));
    }
  }
}

}  // namespace

hipError_t launch_quantize_q4k(const float* x, uint64_t blocks, uint8_t* out, int* failure,
                               hipStream_t s) {
  hipLaunchKernelGGL(quantize_q4k_kernel, dim3(uint32_t((blocks + 31) / 32)), dim3(256), 0, s,
                     x, blocks, out, failure);
  return hipGetLastError();
}

hipError_t launch_quantize_q6k(const float* x, uint64_t blocks, uint8_t* out, hipStream_t s) {
  hipLaunchKernelGGL(quantize_q6k_kernel, dim3(uint32_t((blocks + 15) / 16)), dim3(256), 0, s,
                     x, blocks, out);
  return hipGetLastError();
}

}  // namespace qw38hip
