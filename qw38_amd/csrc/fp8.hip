// FP8 (OCP E4M3FN) path of qw38's prefill and decode (cuda/fp8.hpp, cuda/fp8.cu):
//   pack_fp8    BF16 [m][k] -> E4M3 codes [pm][pk] + FP32 scales [pk/128][pm],
//               one scale per (row, 128-column block) = absmax / 448
//               (cuda/fp8.cu:64-81);
//   fp8 GEMV    y[r] = sum_c value(w[r][c]) * s[c/128][r/128] * x[c], BF16 x,
//               the decode_mmv layout 0x020F (cuda/fp8.cu:82-112, 184-203);
//   fp8 GEMM    y[t][r] = sum over 128-column blocks of sx[b][t] * sw[b][r/128]
//               * sum_c value(x[t][c]) value(w[r][c]) (cuda/fp8.cu:137-160).
//
// The GEMM runs on FP16 MFMAs, not the FP8 ones: on gfx950 the FP8 matrix
// instructions (16x16x32 fp8, 16x16x128 f8f6f4) align the products of a dot
// into a narrow accumulator and lose about 1e-4 of the sum of |products| on
// realistic packed data, while every E4M3 value is exact in FP16 and the FP16
// MFMA keeps the sum to about 1e-7 (the reference's budget is 1e-5 of it,
// tests/fp8_test.cpp:100). Codes are staged in LDS as bytes and widened to
// FP16 per fragment with v_cvt_scalef32_pk_f16_fp8 (scale 1: exact).
#include "lowp.hpp"

namespace qw38hip {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// ---- pack: one block of 128 threads per (row, 128-column block) ----
__global__ __launch_bounds__(128) void pack_fp8_kernel(const uint16_t* __restrict__ x, uint32_t m,
                                                       uint32_t k, uint32_t pm, uint32_t pk,
                                                       uint8_t* __restrict__ codes,
                                                       float* __restrict__ scales) {
  __shared__ float wmax[2];
  const uint32_t r = blockIdx.x, b = blockIdx.y, c = b * 128 + threadIdx.x;
  const float v = (r < m && c < k) ? bf16_to_f32(x[size_t(r) * k + c]) : 0.f;
  float a = isfinite(v) ? fabsf(v) : __builtin_inff();
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
  if ((threadIdx.x & 63u) == 0) wmax[threadIdx.x >> 6] = a;
  __syncthreads();
  const float peak = fmaxf(wmax[0], wmax[1]);
  // nonfinite blocks carry NaN (cuda/fp8.cu:75-77)
  const float scale = isfinite(peak) ? (peak == 0.f ? 1.f : fmaxf(__fdiv_rn(peak, 448.f), 0x1p-126f))
                                     : __builtin_nanf("");
  if (threadIdx.x == 0) scales[size_t(b) * pm + r] = scale;
  codes[size_t(r) * pk + c] = uint8_t(e4m3_rne(__fdiv_rn(v, scale)));
}

// ---- decode GEMV: one wave per row, 16 contiguous codes per lane ----
__device__ __forceinline__ float dot16(const uint4 c, const uint32_t* xw) {
  // codes 16 E4M3 (c), x 16 BF16 as 8 pairs (xw)
  const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float w[4] = {__builtin_amdgcn_cvt_f32_fp8(int(cw[i]), 0), __builtin_amdgcn_cvt_f32_fp8(int(cw[i]), 1),
                        __builtin_amdgcn_cvt_f32_fp8(int(cw[i]), 2), __builtin_amdgcn_cvt_f32_fp8(int(cw[i]), 3)};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t pair = xw[2 * i + (b >> 1)];
      const float xv = __uint_as_float((b & 1) ? (pair & 0xffff0000u) : (pair << 16));
      p = fmaf(w[b], xv, p);
    }
  }
  return p;
}

__global__ __launch_bounds__(256) void fp8_gemv_kernel(const uint8_t* __restrict__ codes,
                                                       const float* __restrict__ scales, uint32_t n,
                                                       uint32_t k, const uint16_t* __restrict__ x,
                                                       void* y, const float* residual, int epi) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  for (uint32_t i = threadIdx.x; i < k; i += 256) xs[i] = x[i];
  __syncthreads();
  const uint32_t lane = threadIdx.x & 63u, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const uint8_t* rp = codes + size_t(row) * k;
  const float* sp = scales + row / 128;
  const uint32_t nb = n / 128;
  float acc = 0.f;
  uint32_t base = lane * 16;
  // two 1 KB rows spans per iteration in flight
  for (; base + 1024 < k; base += 2048) {
    const uint4 c0 = *reinterpret_cast<const uint4*>(rp + base);
    const uint4 c1 = *reinterpret_cast<const uint4*>(rp + base + 1024);
    const float s0 = sp[size_t(base / 128) * nb], s1 = sp[size_t((base + 1024) / 128) * nb];
    const uint4* x0 = reinterpret_cast<const uint4*>(xs + base);
    const uint4* x1 = reinterpret_cast<const uint4*>(xs + base + 1024);
    const uint4 a0 = x0[0], a1 = x0[1], b0 = x1[0], b1 = x1[1];
    const uint32_t xa[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const uint32_t xb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    acc = fmaf(s0, dot16(c0, xa), acc);
    acc = fmaf(s1, dot16(c1, xb), acc);
  }
  if (base < k) {
    const uint4 c0 = *reinterpret_cast<const uint4*>(rp + base);
    const uint4* x0 = reinterpret_cast<const uint4*>(xs + base);
    const uint4 a0 = x0[0], a1 = x0[1];
    const uint32_t xa[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    acc = fmaf(sp[size_t(base / 128) * nb], dot16(c0, xa), acc);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane != 0) return;
  if (epi == QW38_DECODE_STORE_BF16) {
    static_cast<uint16_t*>(y)[row] = f32_to_bf16_rne(acc);
  } else if (epi == QW38_DECODE_RESIDUAL_ADD_FP32) {
    float* dst = y ? static_cast<float*>(y) : const_cast<float*>(residual);
    dst[row] = acc + residual[row];
  } else {
    static_cast<float*>(y)[row] = acc;
  }
}

// ---- GEMM: 128 weight rows x 128 tokens per block, 4 waves of 64 x 64 ----
constexpr uint32_t kStrideB = 144;  // LDS row stride in bytes (128 + 16)

__device__ __forceinline__ half8 widen(uint2 v) {
  const h2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(v.x), 1.f, false);
  const h2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(v.x), 1.f, true);
  const h2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(v.y), 1.f, false);
  const h2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(int(v.y), 1.f, true);
  return half8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__global__ __launch_bounds__(256) void fp8_gemm_kernel(const uint8_t* __restrict__ wc,
                                                       const float* __restrict__ ws, uint32_t n,
                                                       uint32_t k, const uint8_t* __restrict__ xc,
                                                       const float* __restrict__ xsc, uint32_t m,
                                                       void* __restrict__ y,
                                                       const float* __restrict__ residual,
                                                       uint32_t valid, int epi) {
  __shared__ __align__(16) uint8_t Wt[2][128 * kStrideB];
  __shared__ __align__(16) uint8_t Xt[2][128 * kStrideB];
  const uint32_t nbs = n / 128, mbs = m / 128;
  const uint32_t nb = blockIdx.x / mbs, mb = blockIdx.x % mbs;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wr = wave >> 1, wt = wave & 1u, lr = lane & 15u, lk = lane >> 4;
  // staging: thread -> (row sr, 64-byte half sh) of both tiles
  const uint32_t sr = tid >> 1, sh = tid & 1u;
  const uint8_t* wsrc = wc + size_t(nb * 128 + sr) * k + sh * 64;
  const uint8_t* xsrc = xc + size_t(mb * 128 + sr) * k + sh * 64;
  uint4 fw[4], fx[4];
  auto fetch = [&](uint32_t kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fw[i] = *reinterpret_cast<const uint4*>(wsrc + size_t(kb) * 128 + i * 16);
      fx[i] = *reinterpret_cast<const uint4*>(xsrc + size_t(kb) * 128 + i * 16);
    }
  };
  auto store = [&](uint32_t buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<uint4*>(&Wt[buf][sr * kStrideB + sh * 64 + i * 16]) = fw[i];
      *reinterpret_cast<uint4*>(&Xt[buf][sr * kStrideB + sh * 64 + i * 16]) = fx[i];
    }
  };
  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4{0, 0, 0, 0};
  const uint32_t kbs = k / 128;
  fetch(0);
  store(0);
  if (kbs > 1) fetch(1);
  for (uint32_t kb = 0; kb < kbs; ++kb) {
    __syncthreads();  // step kb staged; kb-1 consumed
    const uint32_t buf = kb & 1u;
    if (kb + 1 < kbs) store(buf ^ 1u);
    if (kb + 2 < kbs) fetch(kb + 2);
    f4 P[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) P[i][j] = f4{0, 0, 0, 0};
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {  // 32-column slices of the 128-column block
      half8 af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = widen(*reinterpret_cast<const uint2*>(
            &Wt[buf][(wr * 64 + i * 16 + lr) * kStrideB + q * 32 + lk * 8]));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = widen(*reinterpret_cast<const uint2*>(
            &Xt[buf][(wt * 64 + j * 16 + lr) * kStrideB + q * 32 + lk * 8]));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          P[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], P[i][j], 0, 0, 0);
    }
    // block scales: weight block (kb, nb), token scale of each token tile column
    const float sw = ws[size_t(kb) * nbs + nb];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float s = sw * xsc[size_t(kb) * m + mb * 128 + wt * 64 + j * 16 + lr];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][j][v] = fmaf(s, P[i][j][v], acc[i][j][v]);
    }
  }
  // lane holds rows 4lk..4lk+3 of row tile i for token lr of token tile j.
  // epi 0 writes the raw FP32 product of every padded token (fp8_gemm); the
  // prefill epilogues (cuda/prefill.cu:116-134) write only the first `valid`
  // tokens: BF16 RNE, FP32, or FP32 residual[t][r] + product.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t t = mb * 128 + wt * 64 + j * 16 + lr;
    if (epi != 0 && t >= valid) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = nb * 128 + wr * 64 + i * 16 + lk * 4;
      const size_t o = size_t(t) * n + r;
      float4 v = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      if (epi == QW38_DECODE_STORE_BF16) {
        const uint2 b{uint32_t(f32_to_bf16_rne(v.x)) | (uint32_t(f32_to_bf16_rne(v.y)) << 16),
                      uint32_t(f32_to_bf16_rne(v.z)) | (uint32_t(f32_to_bf16_rne(v.w)) << 16)};
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + o) = b;
        continue;
      }
      if (epi == QW38_DECODE_RESIDUAL_ADD_FP32) {
        const float4 q = *reinterpret_cast<const float4*>(residual + o);
        v = make_float4(q.x + v.x, q.y + v.y, q.z + v.z, q.w + v.w);
      }
      *reinterpret_cast<float4*>(static_cast<float*>(y) + o) = v;
    }
  }
}

__global__ void fp8_store_bf16_kernel(const float* __restrict__ x, uint16_t* __restrict__ y,
                                      uint64_t count) {
  const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < count) y[i] = f32_to_bf16_rne(x[i]);
}

}  // namespace

hipError_t launch_pack_fp8(const uint16_t* x, uint32_t m, uint32_t k, uint8_t* codes, float* scales,
                           hipStream_t s) {
  const uint32_t pm = (m + 127) / 128 * 128, pk = (k + 127) / 128 * 128;
  hipLaunchKernelGGL(pack_fp8_kernel, dim3(pm, pk / 128), dim3(128), 0, s, x, m, k, pm, pk, codes,
                     scales);
  return hipGetLastError();
}

hipError_t launch_fp8_gemv(const uint8_t* codes, const float* scales, uint32_t n, uint32_t k,
                           const uint16_t* x, void* y, const float* residual, int epilogue,
                           hipStream_t s) {
  hipLaunchKernelGGL(fp8_gemv_kernel, dim3((n + 3) / 4), dim3(256), size_t(k) * 2, s, codes,
                     scales, n, k, x, y, residual, epilogue);
  return hipGetLastError();
}

hipError_t launch_fp8_gemm(const uint8_t* wc, const float* ws, uint32_t n, uint32_t k,
                           const uint8_t* xc, const float* xs, uint32_t m, void* y,
                           const float* residual, uint32_t valid, int epilogue, hipStream_t s) {
  hipLaunchKernelGGL(fp8_gemm_kernel, dim3((n / 128) * (m / 128)), dim3(256), 0, s, wc, ws, n, k,
                     xc, xs, m, y, residual, valid, epilogue);
  return hipGetLastError();
}

hipError_t launch_fp8_store_bf16(const float* x, uint16_t* y, uint64_t count, hipStream_t s) {
  hipLaunchKernelGGL(fp8_store_bf16_kernel, dim3(uint32_t((count + 255) / 256)), dim3(256), 0, s, x,
                     y, count);
  return hipGetLastError();
}

}  // namespace qw38hip
