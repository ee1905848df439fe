// Load-time repack of GGML-order super-blocks (row-major, n*(k/256) blocks)
// into the 8-row x K256 tiled layouts. One wave per (row, super-block); the
// byte permutation is lossless (src/format/pack.cpp:216-262 for 0x020D).
#include "common.hpp"

namespace qw38hip {
namespace {

// GGML block_q4_K: d, dmin, scales[12], qs[128] with qs[32j + l] holding codes
// 64j + l (low nibble) and 64j + 32 + l (high nibble).
__device__ __forceinline__ uint32_t q4_code(const uint8_t* blk, uint32_t e) {
  const uint32_t j = e / 64, l = e % 64;
  const uint8_t b = blk[16 + 32 * j + (l % 32)];
  return l < 32 ? (b & 15u) : (b >> 4);
}

__global__ void repack_q4k_kernel(const uint8_t* __restrict__ blocks, uint32_t n, uint32_t kbs,
                                  uint16_t layout, uint8_t* __restrict__ codes,
                                  uint8_t* __restrict__ meta) {
  const uint32_t wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  if (wid >= n * kbs) return;
  const uint32_t row = wid / kbs, kb = wid % kbs;
  const uint8_t* blk = blocks + size_t(wid) * 144;
  const uint64_t tr = (uint64_t(row / 8) * kbs + kb) * 8 + row % 8;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t byte = lane * 2 + h;  // 0..127
    const uint32_t g = byte / 16, j = byte % 16;
    uint32_t lo, hi;
    if (layout == QW38_LAYOUT_Q4K_CANDIDATE_V2) {
      lo = 2 * j;
      hi = 2 * j + 1;
    } else {
      lo = 8 * (j / 4) + (j % 4);
      hi = lo + 4;
    }
    codes[q4k_code_word(layout, row, kb, g, kbs, (n + 7) / 8) + j] =
        uint8_t(q4_code(blk, 32 * g + lo) | (q4_code(blk, 32 * g + hi) << 4));
  }
  if (lane < 16) meta[q4k_meta_row(layout, row, kb, kbs, (n + 7) / 8) + lane] = blk[lane];
}

// GGML block_q6_K: ql[128], qh[64], scales[16], d (fp16 at byte 208).
__device__ __forceinline__ uint32_t q6_code(const uint8_t* y, uint32_t e) {
  const uint32_t half = e / 128, lp = e % 128, part = lp / 32, l = lp % 32;
  const uint8_t* ql = y + 64 * half;
  const uint8_t* qh = y + 128 + 32 * half;
  const uint32_t low = (part & 1) ? ql[l + 32] : ql[l];
  const uint32_t nib = (part & 2) ? (low >> 4) : (low & 15u);
  return nib | (((qh[l] >> (2 * part)) & 3u) << 4);
}

__global__ void repack_q6k_kernel(const uint8_t* __restrict__ blocks, uint32_t n, uint32_t pn,
                                  uint32_t kbs, uint8_t* __restrict__ codes,
                                  uint8_t* __restrict__ meta) {
  const uint32_t wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  if (wid >= n * kbs) return;
  const uint32_t row = wid / kbs, kb = wid % kbs;
  const uint8_t* y = blocks + size_t(wid) * 210;
  const uint64_t tr = (uint64_t(row / 8) * kbs + kb) * 8 + row % 8;
  uint8_t* tile = codes + (tr - row % 8) * kQ6CodeBytes;
  for (uint32_t byte = lane; byte < kQ6CodeBytes; byte += 64) {
    uint32_t v = 0, dst;
    if (byte < 128) {  // (group g, byte j) of the low-nibble chunk
      const uint32_t g = byte / 16, j = byte % 16, t = j / 4, i = j % 4;
      v = (q6_code(y, 32 * g + 8 * t + i) & 15u) | ((q6_code(y, 32 * g + 8 * t + 4 + i) & 15u) << 4);
      dst = q6_chunk(row % 8, g) * 16 + j;
    } else {  // (group g, byte b % 8) of the high-pair chunk
      const uint32_t b = byte - 128, g = b / 8, u = (b % 8) / 4, i = b % 4;
#pragma unroll
      for (uint32_t s = 0; s < 4; ++s)
        v |= ((q6_code(y, 32 * g + 16 * u + 4 * s + i) >> 4) & 3u) << (2 * s);
      dst = kQ6HiPlane + q6_chunk(row % 8, g) * 8 + b % 8;
    }
    tile[dst] = uint8_t(v);
  }
  if (lane < 16) meta[tr * 16 + lane] = y[192 + lane];
  if (lane < 2) meta[uint64_t(pn) * kbs * 16 + tr * 2 + lane] = y[208 + lane];
}

}  // namespace

hipError_t launch_repack_q4k(const uint8_t* blocks, uint32_t n, uint32_t k, uint16_t layout,
                             uint8_t* codes, uint8_t* scales, hipStream_t s) {
  const uint32_t kbs = k / 256;
  const uint64_t waves = uint64_t(n) * kbs;
  hipLaunchKernelGGL(repack_q4k_kernel, dim3(uint32_t((waves + 3) / 4)), dim3(256), 0, s,
                     blocks, n, kbs, layout, codes, scales);
  return hipGetLastError();
}

hipError_t launch_repack_q6k(const uint8_t* blocks, uint32_t n, uint32_t k, uint8_t* codes,
                             uint8_t* scales, hipStream_t s) {
  const uint32_t kbs = k / 256, pn = (n + 7) / 8 * 8;
  const uint64_t waves = uint64_t(n) * kbs;
  hipLaunchKernelGGL(repack_q6k_kernel, dim3(uint32_t((waves + 3) / 4)), dim3(256), 0, s,
                     blocks, n, pn, kbs, codes, scales);
  return hipGetLastError();
}

}  // namespace qw38hip
