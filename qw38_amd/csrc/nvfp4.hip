// NVFP4 path of qw38's prefill and decode (cuda/nvfp4.hpp, cuda/nvfp4.cu,
// cuda/nvfp4_device.cuh, decode_mmv layout 0x020E):
//   pack_nvfp4   BF16 [m][k] -> E2M1 nibbles [m][pk/2] (element 2j in the low
//                nibble of byte j) + UE4M3 block scales of 16 elements in the
//                CUTLASS SM1xx swizzle over 128-row stripes (pad128(m) rows,
//                padding rows' scales 0, padding rows' codes not written);
//   weights      the same element/scale encoding of values / factor, where
//                factor is an FP32 power of two stored in bytes 0..3 of a
//                256-byte header in front of the scales
//                (src/compiler/quantization/nvfp4.cpp:25-56);
//   decode GEMV  BF16 x, weight element RN(RN(scale * factor) * value(code))
//                (cuda/decode_mmv.cu:94-102), FP32 FMAs, optional paired
//                SwiGLU, the decode_mmv epilogues;
//   W4A4 GEMM    y[t][r] = factor * sum_c (sa * a)(sw * w) (cuda/nvfp4.cu:
//                83-116), with the prefill epilogues fused into the store.
//
// The GEMM runs on FP16 MFMAs. gfx950's scaled FP4 MFMA and FP4 conversions
// take E8M0 (power-of-two) scales, and UE4M3 scales are not powers of two.
// But an E2M1 value times a UE4M3 value has at most 5 significant bits and
// lies in [2^-10, 2688], so it is exact in FP16: each operand fragment is
// converted exactly (v_cvt_scalef32_pk_f16_fp4 with scale 1, then a packed
// FP16 multiply by the block scale) and the MFMA chain runs over all of K
// without a per-block rescale. Products of two such FP16 values are exact in
// FP32, so the only rounding is the FP32 accumulation.
#include "lowp.hpp"

namespace qw38hip {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

// ---- activation pack: one block per padded row, one thread per 16-block ----
__global__ __launch_bounds__(128) void pack_nvfp4_kernel(const uint16_t* __restrict__ x,
                                                         uint32_t m, uint32_t k, uint32_t pk,
                                                         uint8_t* __restrict__ codes,
                                                         uint8_t* __restrict__ scales) {
  const uint32_t r = blockIdx.x;
  const bool valid = r < m;
  for (uint32_t b = threadIdx.x; b < pk / 16; b += 128) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t c = b * 16 + i;
      v[i] = valid && c < k ? bf16_to_f32(x[size_t(r) * k + c]) : 0.f;
    }
    uint32_t cw[2];
    const uint32_t s = nvfp4_encode_block(v, cw);
    scales[nvfp4_sf_index(r, b, pk)] = uint8_t(s);
    if (valid) *reinterpret_cast<uint2*>(codes + (size_t(r) * pk + b * 16) / 2) = make_uint2(cw[0], cw[1]);
  }
}

// ---- decode GEMV: one wave per row, 32 contiguous elements per lane ----
// Two consecutive 16-blocks per lane step; their scale bytes are adjacent in
// the swizzle (b even -> b % 4 in {0, 2}). A weight element is
// RN(RN(scale * factor) * value) (cuda/decode_mmv.cu:94-102): the UE4M3 scale
// has at most 4 significant bits and factor is a power of two, so
// scale * factor and its product with an E2M1 value (at most 2 significant
// bits) are exact in FP32. Each block is therefore summed as sum(value * x)
// with exact BF16 operands (v_cvt_scalef32_pk_bf16_fp4, then v_dot2_f32_bf16
// on element pairs) and scaled once: acc += (scale * factor) * block.
__device__ __forceinline__ float nvfp4_dot32(uint4 c, uint32_t sf2, float factor,
                                             const uint32_t (&xw)[16], float acc) {
  typedef __bf16 bfx2 __attribute__((ext_vector_type(2)));
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float sc = __fmul_rn(e4m3_value((sf2 >> (8 * h)) & 0xffu), factor);
    float bs = 0.f;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t word = cw[2 * h + w];
      const bfx2 v[4] = {__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, 1.f, 0),
                         __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, 1.f, 1),
                         __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, 1.f, 2),
                         __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, 1.f, 3)};
#pragma unroll
      for (int bsel = 0; bsel < 4; ++bsel)
        bs = __builtin_amdgcn_fdot2_f32_bf16(v[bsel], __builtin_bit_cast(bfx2, xw[8 * h + 4 * w + bsel]), bs,
                                             false);
    }
    acc = fmaf(sc, bs, acc);
  }
  return acc;
}

__device__ __forceinline__ void decode_store(int epi, void* y, const float* residual, uint32_t row,
                                             float acc) {
  if (epi == QW38_DECODE_STORE_BF16) {
    static_cast<uint16_t*>(y)[row] = f32_to_bf16_rne(acc);
  } else if (epi == QW38_DECODE_RESIDUAL_ADD_FP32) {
    float* dst = y ? static_cast<float*>(y) : const_cast<float*>(residual);
    dst[row] = residual[row] + acc;
  } else {
    static_cast<float*>(y)[row] = acc;
  }
}

// Block: four waves x kRowsPerWave rows. A lane takes 32 contiguous elements
// per step (16 code bytes per row and the 32 BF16 inputs, read from LDS once
// for all the wave's rows); all steps' code and scale loads of a row are
// issued before the first is consumed when K <= 8192.
constexpr uint32_t kRowsPerWave = 4;

template <bool Paired>
__global__ __launch_bounds__(256) void nvfp4_gemv_kernel(
    const uint8_t* __restrict__ ca, const uint8_t* __restrict__ sa, const uint8_t* __restrict__ cb,
    const uint8_t* __restrict__ sb, uint32_t n, uint32_t pn, uint32_t k, uint32_t pk,
    const uint16_t* __restrict__ x, void* ya, void* yb, const float* ra, const float* rb, int epi) {
  constexpr uint32_t R = kRowsPerWave, kMaxSteps = 4, BR = 4 * R;
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  // Scales of the block's BR rows, one dword per (row, quad of blocks): in
  // the swizzle a row's blocks 4q..4q+3 share one aligned dword, and the
  // dwords of consecutive rows are 16 B apart.
  const uint32_t quads = pk / 64;
  uint32_t* sfa_l = reinterpret_cast<uint32_t*>(smem + size_t(pk) * 2);
  uint32_t* sfb_l = sfa_l + BR * quads;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t brow0 = blockIdx.x * BR;  // BR divides 128: the block lies in one stripe
  const uint32_t row0 = brow0 + (threadIdx.x >> 6) * R;
  const uint32_t nsteps = (pk + 2047) / 2048;
  const bool hoist = nsteps <= kMaxSteps;

  // This wave's code loads go out first (rows past pn re-read the last row
  // and are never stored), so they overlap the block's staging below.
  auto load = [&](uint32_t c0, uint4 (&wa)[R], uint4 (&wb)[R]) {
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
      const size_t co = (size_t(min(row0 + r, pn - 1)) * pk + c0) / 2;
      wa[r] = *reinterpret_cast<const uint4*>(ca + co);
      if constexpr (Paired) wb[r] = *reinterpret_cast<const uint4*>(cb + co);
    }
  };
  uint4 wa[kMaxSteps][R], wb[kMaxSteps][R];
  if (hoist && row0 < pn) {
#pragma unroll
    for (uint32_t i = 0; i < kMaxSteps; ++i)
      if (i < nsteps && lane * 32 + i * 2048 < pk) load(lane * 32 + i * 2048, wa[i], wb[i]);
  }

  if ((reinterpret_cast<uintptr_t>(x) % 16) == 0 && k % 8 == 0) {
    for (uint32_t i = threadIdx.x; i < pk / 8; i += 256)
      reinterpret_cast<uint4*>(xs)[i] = 8 * i < k ? reinterpret_cast<const uint4*>(x)[i] : make_uint4(0, 0, 0, 0);
  } else {
    for (uint32_t i = threadIdx.x; i < pk; i += 256) xs[i] = i < k ? x[i] : uint16_t(0);
  }
  for (uint32_t i = threadIdx.x; i < BR * quads; i += 256) {
    const uint32_t rl = i % BR, q = i / BR;
    const uint64_t o = 256 + nvfp4_sf_index(brow0 + rl, 4 * q, pk);
    sfa_l[rl * quads + q] = *reinterpret_cast<const uint32_t*>(sa + o);
    if constexpr (Paired) sfb_l[rl * quads + q] = *reinterpret_cast<const uint32_t*>(sb + o);
  }
  __syncthreads();
  if (row0 >= pn) return;
  const float fa = *reinterpret_cast<const float*>(sa);
  const float fb = Paired ? *reinterpret_cast<const float*>(sb) : 0.f;
  float acc_a[R], acc_b[R];
#pragma unroll
  for (uint32_t r = 0; r < R; ++r) acc_a[r] = acc_b[r] = 0.f;
  auto step = [&](uint32_t c0, const uint4 (&wa_)[R], const uint4 (&wb_)[R]) {
    uint32_t xw[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(xs + c0 + 8 * i);
      xw[4 * i] = v.x; xw[4 * i + 1] = v.y; xw[4 * i + 2] = v.z; xw[4 * i + 3] = v.w;
    }
    const uint32_t sh = 8 * ((c0 / 16) % 4);
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
      const uint32_t li = (row0 + r - brow0) * quads + c0 / 64;
      acc_a[r] = nvfp4_dot32(wa_[r], (sfa_l[li] >> sh) & 0xffffu, fa, xw, acc_a[r]);
      if constexpr (Paired) acc_b[r] = nvfp4_dot32(wb_[r], (sfb_l[li] >> sh) & 0xffffu, fb, xw, acc_b[r]);
    }
  };
  if (hoist) {
#pragma unroll
    for (uint32_t i = 0; i < kMaxSteps; ++i)
      if (i < nsteps && lane * 32 + i * 2048 < pk) step(lane * 32 + i * 2048, wa[i], wb[i]);
  } else {
    for (uint32_t c0 = lane * 32; c0 < pk; c0 += 2048) {
      uint4 ta[R], tb[R];
      load(c0, ta, tb);
      step(c0, ta, tb);
    }
  }
#pragma unroll
  for (uint32_t r = 0; r < R; ++r)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      acc_a[r] += __shfl_xor(acc_a[r], o);
      if constexpr (Paired) acc_b[r] += __shfl_xor(acc_b[r], o);
    }
  if (lane != 0) return;
#pragma unroll
  for (uint32_t r = 0; r < R; ++r) {
    const uint32_t row = row0 + r;
    if (row >= n) break;
    if (Paired && epi == QW38_DECODE_SWIGLU_BF16) {
      static_cast<uint16_t*>(ya)[row] = f32_to_bf16_rne(silu(acc_a[r]) * acc_b[r]);
      continue;
    }
    decode_store(epi, ya, ra, row, acc_a[r]);
    if constexpr (Paired) decode_store(epi, yb, rb, row, acc_b[r]);
  }
}

// ---- W4A4 GEMM: 128 weight rows x 128 tokens per block, 4 waves of 64 x 64 ----
constexpr uint32_t kCodeStride = 80;  // LDS bytes per 128-element row of nibbles (64 + 16)

struct Operand {
  const uint8_t* codes;   // row-major nibbles, row stride pk/2
  const uint8_t* scales;  // swizzled UE4M3 of this operand's 128-row stripes
  uint32_t rows;          // rows with codes (reads beyond are zero)
};

// fragment of the 16x16x32 f16 MFMA: 8 consecutive elements of one row,
// exact FP16 value * block scale
__device__ __forceinline__ half8 widen4(uint32_t w, _Float16 s) {
  const h2 ss{s, s};
  const h2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.f, 0) * ss;
  const h2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.f, 1) * ss;
  const h2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.f, 2) * ss;
  const h2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.f, 3) * ss;
  return half8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Scale of (row r, block j) of a staged 128 x 8-block chunk (the 1 KB of the
// swizzle that covers it, converted to FP16).
__device__ __forceinline__ uint32_t chunk_sf(uint32_t r, uint32_t j) {
  return (j / 4) * 512 + (r % 32) * 16 + (r / 32) * 4 + j % 4;
}

// epi 0 writes factor * sum as FP32 [m][n]; the decode epilogue IDs write
// the prefill epilogues (cuda/prefill.cu:116-134); kSwiglu writes
// BF16(SiLU(gate[t][r]) * (factor * sum)) with the gate projection read from
// `residual` (FP32 [m][n], an earlier epi-0 launch), the paired order of
// cuda/prefill.cu:203-215.
constexpr int kSwiglu = QW38_DECODE_SWIGLU_BF16;

__global__ __launch_bounds__(256) void nvfp4_gemm_kernel(Operand wo, const float* __restrict__ fp,
                                                         uint32_t n, uint32_t pk, Operand xa,
                                                         uint32_t m, void* __restrict__ y,
                                                         const float* __restrict__ residual,
                                                         int epi) {
  __shared__ __align__(16) uint8_t Ct[2][2][128 * kCodeStride];
  __shared__ __align__(16) _Float16 St[2][2][1024];
  const float factor = *fp;  // global weight factor
  const uint32_t mbs = (m + 127) / 128;
  const uint32_t nb = blockIdx.x / mbs, mb = blockIdx.x % mbs;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wr = wave >> 1, wt = wave & 1u, lr = lane & 15u, lk = lane >> 4;
  // operand 0: weights (rows nb*128..), operand 1: activations (tokens mb*128..)
  const Operand ops[2] = {wo, xa};
  const uint32_t base_row[2] = {nb * 128, mb * 128};
  // staging: codes thread -> (row sr, 32-byte half sh); scales: 64 threads x 16 B per operand
  const uint32_t sr = tid >> 1, sh = tid & 1u;
  const uint32_t so = tid >> 6, sq = tid & 63u;
  uint4 fc[2][2], fs = make_uint4(0, 0, 0, 0);
  auto fetch = [&](uint32_t kc) {
    // Branch-free: rows without codes load a clamped row and are zeroed by a
    // select (a branch around these carried prefetches also crashes this
    // compiler's machine copy propagation).
#pragma unroll
    for (int o = 0; o < 2; ++o) {
      const uint32_t row = base_row[o] + sr;
      const bool live = row < ops[o].rows;
      const uint32_t rr = live ? row : ops[o].rows - 1;
      const uint4* p = reinterpret_cast<const uint4*>(ops[o].codes + (size_t(rr) * pk + kc * 128) / 2 + sh * 32);
      const uint4 c0 = p[0], c1 = p[1];
      const uint4 z = make_uint4(0, 0, 0, 0);
      fc[o][0] = live ? c0 : z;
      fc[o][1] = live ? c1 : z;
    }
    const uint32_t os = so & 1u;  // waves 2, 3 repeat the activation scales; only 0, 1 store
    fs = *reinterpret_cast<const uint4*>(ops[os].scales + size_t(base_row[os] / 128) * 128 * (pk / 16) +
                                        size_t(kc) * 1024 + sq * 16);
  };
  auto store = [&](uint32_t buf) {
#pragma unroll
    for (int o = 0; o < 2; ++o) {
      *reinterpret_cast<uint4*>(&Ct[buf][o][sr * kCodeStride + sh * 32]) = fc[o][0];
      *reinterpret_cast<uint4*>(&Ct[buf][o][sr * kCodeStride + sh * 32 + 16]) = fc[o][1];
    }
    if (so < 2) {
      const uint32_t b[4] = {fs.x, fs.y, fs.z, fs.w};
      _Float16 h[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) h[i] = _Float16(e4m3_value((b[i / 4] >> (8 * (i % 4))) & 0xffu));
      uint4* d = reinterpret_cast<uint4*>(&St[buf][so][sq * 16]);
      d[0] = *reinterpret_cast<const uint4*>(&h[0]);
      d[1] = *reinterpret_cast<const uint4*>(&h[8]);
    }
  };
  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4{0, 0, 0, 0};
  const uint32_t kcs = pk / 128;
  fetch(0);
  store(0);
  if (kcs > 1) fetch(1);
  for (uint32_t kc = 0; kc < kcs; ++kc) {
    __syncthreads();  // chunk kc staged; kc-1 consumed
    const uint32_t buf = kc & 1u;
    if (kc + 1 < kcs) store(buf ^ 1u);
    if (kc + 2 < kcs) fetch(kc + 2);
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {  // 32-element slices of the 128-element chunk
      const uint32_t kk = q * 32 + lk * 8, j = kk / 16;
      half8 af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t r = wr * 64 + i * 16 + lr;
        af[i] = widen4(*reinterpret_cast<const uint32_t*>(&Ct[buf][0][r * kCodeStride + kk / 2]),
                       St[buf][0][chunk_sf(r, j)]);
      }
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const uint32_t t = wt * 64 + jt * 16 + lr;
        bf[jt] = widen4(*reinterpret_cast<const uint32_t*>(&Ct[buf][1][t * kCodeStride + kk / 2]),
                        St[buf][1][chunk_sf(t, j)]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
          acc[i][jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[jt], acc[i][jt], 0, 0, 0);
    }
  }
  // lane holds rows 4lk..4lk+3 of row tile i for token lr of token tile jt
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    const uint32_t t = mb * 128 + wt * 64 + jt * 16 + lr;
    if (t >= m) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = nb * 128 + wr * 64 + i * 16 + lk * 4;
      if (r >= n) continue;  // n % 8 == 0: whole 4-row groups
      const size_t o = size_t(t) * n + r;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = factor * acc[i][jt][e];
      if (epi == kSwiglu) {
        const float4 g = *reinterpret_cast<const float4*>(residual + o);
        const uint2 b{uint32_t(f32_to_bf16_rne(silu(g.x) * v[0])) |
                          (uint32_t(f32_to_bf16_rne(silu(g.y) * v[1])) << 16),
                      uint32_t(f32_to_bf16_rne(silu(g.z) * v[2])) |
                          (uint32_t(f32_to_bf16_rne(silu(g.w) * v[3])) << 16)};
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + o) = b;
        continue;
      }
      if (epi == QW38_DECODE_STORE_BF16) {
        const uint2 b{uint32_t(f32_to_bf16_rne(v[0])) | (uint32_t(f32_to_bf16_rne(v[1])) << 16),
                      uint32_t(f32_to_bf16_rne(v[2])) | (uint32_t(f32_to_bf16_rne(v[3])) << 16)};
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + o) = b;
        continue;
      }
      if (epi == QW38_DECODE_RESIDUAL_ADD_FP32) {
        const float4 q = *reinterpret_cast<const float4*>(residual + o);
        v[0] = q.x + v[0];
        v[1] = q.y + v[1];
        v[2] = q.z + v[2];
        v[3] = q.w + v[3];
      }
      *reinterpret_cast<float4*>(static_cast<float*>(y) + o) = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

}  // namespace

hipError_t launch_pack_nvfp4(const uint16_t* x, uint32_t m, uint32_t k, uint8_t* codes,
                             uint8_t* scales, hipStream_t s) {
  const uint32_t pk = (k + 255) / 256 * 256;
  hipLaunchKernelGGL(pack_nvfp4_kernel, dim3((m + 127) / 128 * 128), dim3(128), 0, s, x, m, k, pk,
                     codes, scales);
  return hipGetLastError();
}

hipError_t launch_nvfp4_gemv(const uint8_t* ca, const uint8_t* sa, const uint8_t* cb,
                             const uint8_t* sb, uint32_t n, uint32_t pn, uint32_t k, uint32_t pk,
                             const uint16_t* x, void* ya, void* yb, const float* ra, const float* rb,
                             int epilogue, hipStream_t s) {
  const dim3 grid((pn + 4 * kRowsPerWave - 1) / (4 * kRowsPerWave));
  const size_t lds = size_t(pk) * 2 + size_t(2) * 4 * kRowsPerWave * (pk / 64) * 4;
  if (cb)
    hipLaunchKernelGGL(nvfp4_gemv_kernel<true>, grid, dim3(256), lds, s, ca, sa, cb, sb, n,
                       pn, k, pk, x, ya, yb, ra, rb, epilogue);
  else
    hipLaunchKernelGGL(nvfp4_gemv_kernel<false>, grid, dim3(256), lds, s, ca, sa, cb, sb,
                       n, pn, k, pk, x, ya, yb, ra, rb, epilogue);
  return hipGetLastError();
}

hipError_t launch_nvfp4_gemm(const uint8_t* wc, const uint8_t* wsf, const float* wfactor,
                             uint32_t n, uint32_t code_rows, uint32_t pk, const uint8_t* xc,
                             const uint8_t* xs, uint32_t m, void* y, const float* residual,
                             int epilogue, hipStream_t s) {
  const Operand w{wc, wsf, code_rows}, x{xc, xs, m};
  const dim3 grid(((n + 127) / 128) * ((m + 127) / 128));
  hipLaunchKernelGGL(nvfp4_gemm_kernel, grid, dim3(256), 0, s, w, wfactor, n, pk, x, m, y, residual,
                     epilogue);
  return hipGetLastError();
}

}  // namespace qw38hip
