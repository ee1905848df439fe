// Low-precision element formats shared by the FP8 and NVFP4 kernels and the
// fused RMS producers:
//   E4M3FN  (OCP FP8: bias 7, subnormals, no infinities, 0x7F/0xFF NaN);
//   UE4M3   (the unsigned NVFP4 block scale: E4M3 codes 0..126, 127 NaN);
//   E2M1    (the NVFP4 element: {0, .5, 1, 1.5, 2, 3, 4, 6} and sign bit 3).
// Encoders round to nearest with ties to the even code, which is what the
// reference's exhaustive nearest-value encoder of tests/nvfp4_test.cpp:47-56
// and tests/fp8_test.cpp:34-43 defines; both code sequences are monotone in
// value, so nearest-even is RNE on the exponent/mantissa split with
// saturation at the largest finite code.
#pragma once

#include "common.hpp"

namespace qw38hip {

// E4M3FN, finite values saturating at +-448, NaN -> 0x7F.
__device__ __forceinline__ uint32_t e4m3_rne(float x) {
  if (x != x) return 0x7Fu;
  const uint32_t s = (__float_as_uint(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  if (a >= 448.f) return s | 0x7Eu;
  if (a < 0.015625f) return s | uint32_t(rintf(a * 512.f));  // multiples of 2^-9
  const uint32_t b = __float_as_uint(a);
  const uint32_t r = b + 0x7ffffu + ((b >> 20) & 1u);  // 3-bit mantissa, half to even
  const int e = int(r >> 23) - 127;
  const uint32_t mm = (r >> 20) & 7u;
  if (e > 8 || (e == 8 && mm == 7)) return s | 0x7Eu;
  return s | (uint32_t(e + 7) << 3) | mm;
}

// Value of an E4M3 code; for codes 0..127 this is the UE4M3 block scale
// (127 -> NaN).
__device__ __forceinline__ float e4m3_value(uint32_t c) {
  return __builtin_amdgcn_cvt_f32_fp8(int(c), 0);
}

// E2M1 magnitude code of |q| (0..7): nearest of {0,.5,1,1.5,2,3,4,6}, ties
// to the even code, saturating at 6.
__device__ __forceinline__ uint32_t e2m1_magnitude(float a) {
  return a <= 0.25f ? 0u : a < 0.75f ? 1u : a <= 1.25f ? 2u : a < 1.75f ? 3u
       : a <= 2.5f ? 4u : a < 3.5f ? 5u : a <= 5.f ? 6u : 7u;
}

// NVFP4 block-scale position: CUTLASS's SM1xx K-major scale-factor atom of
// 128 rows x 4 blocks (src/format/nvfp4.hpp:14-17, cuda/nvfp4_device.cuh:
// 6-10). 128-row stripes of pk/16 bytes; inside a stripe, groups of four
// 16-element blocks are 512-byte chunks indexed by (row%32, row/32%4, b%4).
__device__ __forceinline__ uint64_t nvfp4_sf_index(uint32_t row, uint32_t block, uint32_t pk) {
  return uint64_t(row / 128) * 128 * (pk / 16) + (block / 4) * 512 + (row % 32) * 16 +
         ((row % 128) / 32) * 4 + block % 4;
}

// One NVFP4 block of 16 values (cuda/nvfp4_device.cuh:18-49 for activations,
// src/compiler/quantization/nvfp4.cpp:37-56 for weights after the global
// factor): scale code = UE4M3(peak / 6) (1 if that rounds to 0 for a nonzero
// peak; 127 for a block holding a nonfinite value), element code =
// E2M1(v / scale) with the sign of v, 0 for v == 0 and for nonfinite blocks.
// Returns the scale code; codes[i] holds the 16 nibbles, element 2j in the
// low nibble of byte j.
__device__ __forceinline__ uint32_t nvfp4_encode_block(const float v[16], uint32_t codes[2]) {
  float peak = 0.f;
  bool finite = true;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    finite &= isfinite(v[i]);
    peak = fmaxf(peak, fabsf(v[i]));
  }
  uint32_t s = finite ? e4m3_rne(__fdiv_rn(peak, 6.f)) : 127u;
  if (peak != 0.f && s == 0u) s = 1u;
  const float scale = e4m3_value(s);
  codes[0] = codes[1] = 0u;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint32_t c = 0u;
    if (finite && v[i] != 0.f) {
      const float q = __fdiv_rn(v[i], scale);
      c = e2m1_magnitude(fabsf(q)) | ((__float_as_uint(q) >> 28) & 8u);
    }
    codes[i / 8] |= c << (4 * (i % 8));
  }
  return s;
}

}  // namespace qw38hip
