// Q8 activation producers for gfx950: standalone BF16 pack, fused RMS->Q8 and
// fused SwiGLU->Q8. One K32 group is one 32-lane half of a wave64; the group
// reductions stay inside that half (width-32 shuffles, one ballot).
//
// Semantics (bit-exact): cuda/q8_device.cuh:6-25 -- peak = max finite |x|,
// a = peak == 0 ? 1 : RN(peak / 127), z = clamp(rint(RN(x / a)), -127, 127),
// sum = sum z; a nonfinite group stores a = NaN, z = 0 and raises the flag.
#include "lowp.hpp"

namespace qw38hip {
namespace {

// cuda/q4k_q8.cu:44-50: grid (pk/256, m); padding columns pack as zeros.
__global__ __launch_bounds__(256) void pack_q8_kernel(const uint16_t* __restrict__ in,
                                                      uint32_t k, uint32_t pk,
                                                      int8_t* codes, float* scales,
                                                      int32_t* sums, int* failure) {
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  const uint32_t row = blockIdx.y;
  const float x = c < k ? bf16_to_f32(in[size_t(row) * k + c]) : 0.f;
  q8_group32(x, codes, scales, sums, (size_t(row) * pk + c) / 32, failure);
}

__device__ __forceinline__ float tree32_max(float v) {
#pragma unroll
  for (int off = 16; off; off >>= 1) v = fmaxf(v, __shfl_down(v, off, 32));
  return v;
}
// 256-thread block reduction in the reference's order (cuda/activation.cu:
// 52-96): eight 32-lane trees, then one tree over the 8 partials + 24 zeros.
template <bool Max>
__device__ float block256(float v, float* sm) {
  v = Max ? tree32_max(v) : tree32_sum(v);
  const unsigned w32 = threadIdx.x >> 5, lane = threadIdx.x & 31u;
  if (lane == 0) sm[w32] = v;
  __syncthreads();
  if (threadIdx.x < 32) {
    float t = lane < 8 ? sm[lane] : 0.f;
    t = Max ? tree32_max(t) : tree32_sum(t);
    if (lane == 0) sm[8] = t;
  }
  __syncthreads();
  float r = sm[8];
  __syncthreads();
  return r;
}

constexpr uint32_t kHidden = 5120;

// cuda/activation.cu:134-190: absmax prescale, sum of squares,
// (1+gamma)*x/rms -> BF16 RNE, then by Mode:
//   kRmsBf16   the BF16 row is the output (hidden_rms_kernel<0>);
//   (the Q8 pack of the BF16 row, hidden_rms_kernel<3>, is rms_q8_wide_kernel)
//   kRmsNvfp4  NVFP4 pack (hidden_rms_kernel<1>, cuda/nvfp4_device.cuh:18-49);
//   kRmsFp8    FP8 pack into codes [pm][5120] / scales [40][pm], the BF16 row
//              also stored when out_bf16 is given (hidden_rms_kernel<2>,
//              cuda/fp8_device.cuh:8-26).
// NVFP4/FP8 grids cover pad128(m) rows; padding rows only write their
// padding scales (NVFP4: 0; FP8: scale 1 and zero codes).
// FMAs where nvcc contracts mul+add.
enum RmsMode { kRmsBf16 = 0, kRmsQ8 = 1, kRmsNvfp4 = 2, kRmsFp8 = 3 };

// one 128-element FP8 block per wave: two elements per lane
__device__ __forceinline__ void fp8_block128(float v0, float v1, uint32_t r, uint32_t b, uint32_t pm,
                                             uint8_t* codes, float* scales) {
  float peak = fmaxf(isfinite(v0) ? fabsf(v0) : __builtin_inff(), isfinite(v1) ? fabsf(v1) : __builtin_inff());
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) peak = fmaxf(peak, __shfl_xor(peak, o));
  const float scale = isfinite(peak) ? (peak == 0.f ? 1.f : fmaxf(__fdiv_rn(peak, 448.f), 0x1p-126f))
                                     : __builtin_nanf("");
  const uint32_t lane = threadIdx.x & 63u;
  if (lane == 0) scales[size_t(b) * pm + r] = scale;
  codes[size_t(r) * kHidden + b * 128 + lane] = uint8_t(e4m3_rne(__fdiv_rn(v0, scale)));
  codes[size_t(r) * kHidden + b * 128 + 64 + lane] = uint8_t(e4m3_rne(__fdiv_rn(v1, scale)));
}

template <int Mode>
__global__ __launch_bounds__(256) void rms_kernel(const float* __restrict__ residual,
                                                  const uint16_t* __restrict__ gamma, float eps,
                                                  uint16_t* out_bf16, uint32_t m, uint8_t* codes,
                                                  float* scales, int32_t* sums, int* failure,
                                                  uint8_t* sf_bytes) {
  if constexpr (Mode == kRmsNvfp4 || Mode == kRmsFp8) {
    if (blockIdx.x >= m) {
      if constexpr (Mode == kRmsNvfp4) {
        for (uint32_t b = threadIdx.x; b < kHidden / 16; b += 256)
          sf_bytes[nvfp4_sf_index(blockIdx.x, b, kHidden)] = 0;
      } else {
        for (uint32_t b = threadIdx.x >> 6; b < kHidden / 128; b += 4)
          fp8_block128(0.f, 0.f, blockIdx.x, b, gridDim.x, codes, scales);
      }
      return;
    }
  }
  // Thread t owns elements t + 256 j (j < 20), held in registers: one round
  // of loads for the whole row, the per-thread sums run in increasing j (the
  // order of the strided loops of the reference kernel).
  constexpr int kPer = kHidden / 256;
  constexpr bool Lds = Mode == kRmsNvfp4 || Mode == kRmsFp8;
  __shared__ __align__(16) uint16_t rounded[Lds ? kHidden : 1];
  __shared__ float sm[9];
  const float* x = residual + size_t(blockIdx.x) * kHidden;
  float xv[kPer], gv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    xv[j] = x[threadIdx.x + 256 * j];
    gv[j] = bf16_to_f32(gamma[threadIdx.x + 256 * j]);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) s = fmaxf(s, fabsf(xv[j]));
  const float scale = block256<true>(s, sm);
  const float safe = scale == 0.f ? 1.f : scale;
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    xv[j] = xv[j] / safe;
    sq = fmaf(xv[j], xv[j], sq);
  }
  const float sumsq = block256<false>(sq, sm);
  const float se = sqrtf(eps) / safe;
  const float inv = 1.0f / sqrtf(fmaf(se, se, sumsq / float(kHidden)));
  uint16_t yv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const uint32_t i = threadIdx.x + 256 * j;
    yv[j] = f32_to_bf16_rne((1.0f + gv[j]) * (xv[j] * inv));
    if constexpr (Mode == kRmsBf16) out_bf16[size_t(blockIdx.x) * kHidden + i] = yv[j];
    if constexpr (Lds) rounded[i] = yv[j];
    if constexpr (Mode == kRmsFp8)
      if (out_bf16) out_bf16[size_t(blockIdx.x) * kHidden + i] = yv[j];
  }
  if constexpr (Lds) {
    __syncthreads();
    if constexpr (Mode == kRmsNvfp4) {
      for (uint32_t b = threadIdx.x; b < kHidden / 16; b += 256) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = bf16_to_f32(rounded[b * 16 + i]);
        uint32_t cw[2];
        sf_bytes[nvfp4_sf_index(blockIdx.x, b, kHidden)] = uint8_t(nvfp4_encode_block(v, cw));
        *reinterpret_cast<uint2*>(codes + (size_t(blockIdx.x) * kHidden + b * 16) / 2) = make_uint2(cw[0], cw[1]);
      }
    } else {
      const uint32_t lane = threadIdx.x & 63u;
      for (uint32_t b = threadIdx.x >> 6; b < kHidden / 128; b += 4)
        fp8_block128(bf16_to_f32(rounded[b * 128 + lane]), bf16_to_f32(rounded[b * 128 + 64 + lane]),
                     blockIdx.x, b, gridDim.x, codes, scales);
    }
  }
}

// RMS -> Q8 with 16 waves per row (rms_q8_row in common.hpp).
__global__ __launch_bounds__(1024) void rms_q8_wide_kernel(const float* __restrict__ residual,
                                                           const uint16_t* __restrict__ gamma, float eps,
                                                           int8_t* codes, float* scales, int32_t* sums,
                                                           int* failure, int clear_failure) {
  __shared__ float sm[18];
  __shared__ float xs[kRmsHidden];
  const size_t row = blockIdx.x;
  // one-block grid: the flag is cleared before the row's barriers, so every
  // store that sets it comes after (plain vector store)
  if (clear_failure && threadIdx.x == 0) *failure = 0;
  rms_q8_row<1024>(residual + row * kRmsHidden, gamma, eps, codes + row * kRmsHidden,
                   scales + row * (kRmsHidden / 32), sums + row * (kRmsHidden / 32), failure, sm, xs);
}

// cuda/q4k_q8.cu:52-61: v = BF16(SiLU(g) * u); nonfinite g/u -> NaN -> flag.
__global__ __launch_bounds__(256) void swiglu_q8_kernel(const float* __restrict__ gate,
                                                        const float* __restrict__ up,
                                                        int8_t* codes, float* scales,
                                                        int32_t* sums, int* failure) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  q8_group32(swiglu_q8_value(gate[i], up[i]), codes, scales, sums, i / 32, failure);
}

__global__ void fill_zero_i32_kernel(int* p, uint32_t count) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = 0;
}

}  // namespace

hipError_t launch_pack_q8(const uint16_t* in, uint32_t m, uint32_t k, uint32_t pk,
                          int8_t* codes, float* scales, int32_t* sums, int* failure,
                          hipStream_t s) {
  hipLaunchKernelGGL(pack_q8_kernel, dim3(pk / 256, m), dim3(256), 0, s, in, k, pk, codes,
                     scales, sums, failure);
  return hipGetLastError();
}

hipError_t launch_rms_q8(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                         int8_t* codes, float* scales, int32_t* sums, int* failure,
                         hipStream_t s, bool clear_failure) {
  if (clear_failure && m != 1) return hipErrorInvalidValue;  // other blocks could set it first
  hipLaunchKernelGGL(rms_q8_wide_kernel, dim3(m), dim3(1024), 0, s, residual, gamma, eps, codes, scales, sums,
                     failure, clear_failure ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_rms_bf16(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                           uint16_t* out, hipStream_t s) {
  hipLaunchKernelGGL(rms_kernel<kRmsBf16>, dim3(m), dim3(256), 0, s, residual, gamma, eps, out, m,
                     nullptr, nullptr, nullptr, nullptr, nullptr);
  return hipGetLastError();
}

hipError_t launch_rms_nvfp4(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                            uint8_t* codes, uint8_t* scales, hipStream_t s) {
  hipLaunchKernelGGL(rms_kernel<kRmsNvfp4>, dim3((m + 127) / 128 * 128), dim3(256), 0, s, residual,
                     gamma, eps, nullptr, m, codes, nullptr, nullptr, nullptr, scales);
  return hipGetLastError();
}

hipError_t launch_rms_fp8(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                          uint16_t* companion, uint8_t* codes, float* scales, hipStream_t s) {
  hipLaunchKernelGGL(rms_kernel<kRmsFp8>, dim3((m + 127) / 128 * 128), dim3(256), 0, s, residual,
                     gamma, eps, companion, m, codes, scales, nullptr, nullptr, nullptr);
  return hipGetLastError();
}

hipError_t launch_swiglu_q8(const float* gate, const float* up, uint32_t m, uint32_t n,
                            int8_t* codes, float* scales, int32_t* sums, int* failure,
                            hipStream_t s) {
  const uint64_t total = uint64_t(m) * n;
  hipLaunchKernelGGL(swiglu_q8_kernel, dim3(uint32_t(total / 256)), dim3(256), 0, s, gate, up,
                     codes, scales, sums, failure);
  return hipGetLastError();
}

hipError_t launch_fill_zero_i32(int* p, uint32_t count, hipStream_t s) {
  hipLaunchKernelGGL(fill_zero_i32_kernel, dim3((count + 255) / 256), dim3(256), 0, s, p,
                     count);
  return hipGetLastError();
}

}  // namespace qw38hip
