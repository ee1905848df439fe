// Shared device helpers and internal launch interfaces of the gfx950 kernels.
// Host code (capi.cpp) includes this header for the launcher declarations.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "qw38_hip.h"

namespace qw38hip {

// 8-row x K256 tiles (src/format/pack.cpp:216-262): tile row index of
// (row, kb) and the per-tile-row byte counts of each layout.
constexpr uint32_t kTileRows = 8;
constexpr uint32_t kTileK = 256;
constexpr uint32_t kQ4CodeBytes = 128;  // per tile row
constexpr uint32_t kQ4MetaBytes = 16;
constexpr uint32_t kQ6CodeBytes = 192;  // 128 low-nibble + 64 high-pair bytes
constexpr uint32_t kQ6ScaleBytes = 16;  // + 2 B fp16 d in a trailing array
// Q6_K 0x0241 code planes: an 8-row tile (strip, kb) is 1536 contiguous bytes
// at (strip * kbs + kb) * 1536, the 1024-byte low-nibble plane (16 B per
// (row r, K32 group g)) followed by the 512-byte high-pair plane (8 B each),
// both indexed by chunk q6_chunk(r, g): the two groups of a pair sit side by
// side for each row, and one chunk per lane of a wave covers a whole plane.
constexpr uint32_t kQ6TileBytes = 1536;
constexpr uint32_t kQ6HiPlane = 1024;
__host__ __device__ constexpr uint32_t q6_chunk(uint32_t r, uint32_t g) {
  return (g >> 1) * 16 + 2 * r + (g & 1);
}

struct Q8View {
  const int8_t* codes;
  const float* scales;
  const int32_t* sums;
  uint32_t m, k, pk;
};

struct WeightView {
  const uint8_t* codes;
  const uint8_t* scales;
  uint16_t layout;
  uint32_t n, k, pn, pk;
};

// ---- device scalar helpers -------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(uint32_t(h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
  uint32_t b = __float_as_uint(x);
  if (((b >> 23) & 0xffu) == 0xffu) {
    uint16_t h = uint16_t(b >> 16);
    if (b & 0x7fffffu) h |= 0x40u;
    return h;
  }
  return uint16_t((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
// Exact FP16 -> FP32 (v_cvt_f32_f16; FP16 denormals are preserved by the
// default gfx9 float mode).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return float(__builtin_bit_cast(_Float16, uint16_t(h)));
}

// v_perm_b32: bytes of {hi:lo} selected by sel (0-3 from lo, 4-7 from hi).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(int(a), int(b), c, false);
}

// Q4_K 6-bit scale/min of K32 group g from the three packed metadata words
// p0 = bytes 4..7, p1 = 8..11, p2 = 12..15 of the 16-byte tile-row metadata
// (reference get_scale_min_k4, third_party/llama.cpp-q4k/reference.hpp:174-181).
__device__ __forceinline__ void q4k_scale_min(uint32_t p0, uint32_t p1, uint32_t p2,
                                              uint32_t g, uint32_t& s, uint32_t& m) {
  if (g < 4) {
    s = (p0 >> (8 * g)) & 63u;
    m = (p1 >> (8 * g)) & 63u;
  } else {
    uint32_t j = 8 * (g - 4);
    s = ((p2 >> j) & 15u) | (((p0 >> (j + 6)) & 3u) << 4);
    m = ((p2 >> (j + 4)) & 15u) | (((p1 >> (j + 6)) & 3u) << 4);
  }
}

// Branch-free (v_bfe + selects) 6-bit scale/min extraction for a lane-varying group g.
__device__ __forceinline__ void q4_scale_min_lane(uint32_t p0, uint32_t p1, uint32_t p2,
                                                  uint32_t g, float& s, float& m) {
  const bool hi = g >= 4;
  const uint32_t sh = 8u * (g & 3u);
  const uint32_t width = hi ? 4u : 6u;
  const uint32_t hmask = hi ? 0x30u : 0u;
  const uint32_t sl = __builtin_amdgcn_ubfe(hi ? p2 : p0, sh, width);
  const uint32_t ml = __builtin_amdgcn_ubfe(hi ? p2 : p1, hi ? sh + 4u : sh, width);
  const uint32_t sh2 = (__builtin_amdgcn_ubfe(p0, sh + 6u, 2u) << 4) & hmask;
  const uint32_t mh2 = (__builtin_amdgcn_ubfe(p1, sh + 6u, 2u) << 4) & hmask;
  s = float(sl | sh2);
  m = float(ml | mh2);
}

// exp(x) by Cody-Waite reduction and a degree-7 Taylor polynomial with explicit
// FMAs (Cephes two-part ln2). Within 1 ulp of the correctly rounded result.
__device__ __forceinline__ float exp_cw(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_inff();
  if (x < -103.972084045410f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.98412698412698412698e-4f;
  p = fmaf(p, r, 1.38888888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, int(n));
}

// SiLU with the logistic sigmoid in the reference's two-branch form
// (cuda/decode_mmv.cu:78-85, cuda/prefill.cu:136-141) on exp_cw.
__device__ __forceinline__ float silu(float z) {
  float sg;
  if (z >= 0.f) {
    sg = 1.f / (1.f + exp_cw(-z));
  } else {
    const float e = exp_cw(z);
    sg = e / (1.f + e);
  }
  return z * sg;
}

// Q8 MLP producer value (cuda/q4k_q8.cu:52-61): BF16(SiLU(g) * u) with the
// plain g / (1 + e^-g) form, widened back to FP32; nonfinite g or u give NaN.
__device__ __forceinline__ float swiglu_q8_value(float g, float u) {
  float v = (g / (1.f + exp_cw(-g))) * u;
  if (!isfinite(g) || !isfinite(u)) v = __uint_as_float(0x7fc00000u);
  return bf16_to_f32(f32_to_bf16_rne(v));
}

// Q8 K32 group pack (cuda/q8_device.cuh:6-25): peak = max finite |x|,
// a = peak == 0 ? 1 : RN(peak / 127), z = clamp(rint(RN(x / a)), -127, 127),
// sum = sum z; a nonfinite group stores a = NaN, z = 0 and raises the flag.
// One K32 group per 32-lane half of a wave64 (lane = threadIdx.x % 32; the
// reductions stay inside the half). `active` false: the half takes part in
// the shuffles but stores nothing.
__device__ __forceinline__ void q8_group32(float x, int8_t* codes, float* scales,
                                           int32_t* sums, size_t group, int* failure,
                                           bool active = true) {
  const unsigned lane = threadIdx.x & 31u;
  const bool finite = isfinite(x);
  float peak = finite ? fabsf(x) : 0.f;
#pragma unroll
  for (int off = 16; off; off >>= 1) peak = fmaxf(peak, __shfl_xor(peak, off, 32));
  const uint64_t ballot = __ballot(finite);
  const uint32_t half = uint32_t(ballot >> (threadIdx.x & 32u));
  const float a = peak == 0.f ? 1.f : peak / 127.f;
  const bool valid = half == 0xffffffffu && isfinite(a) && a > 0.f;
  int z = 0;
  if (valid) z = max(-127, min(127, int(rintf(x / a))));
  if (active) codes[group * 32 + lane] = int8_t(z);
  int sum = z;
#pragma unroll
  for (int off = 16; off; off >>= 1) sum += __shfl_xor(sum, off, 32);
  if (active && lane == 0) {
    scales[group] = valid ? a : __uint_as_float(0x7fc00000u);
    sums[group] = sum;
    if (!valid) *failure = 1;  // sticky flag, plain vector store
  }
}

// 32-lane shuffle-down tree (lane i += lane i+off), result valid in lane 0 of
// each half: the warp-32 order of cuda/activation.cu:36-50.
__device__ __forceinline__ float tree32_sum(float v) {
#pragma unroll
  for (int off = 16; off; off >>= 1) v += __shfl_down(v, off, 32);
  return v;
}

constexpr uint32_t kRmsHidden = 5120;

// RMS -> BF16 -> Q8 of one 5120-element row by a block of NT threads (512 or
// 1024): cuda/activation.cu:134-190 with the Q8 pack of hidden_rms_kernel<3>.
// The sum of squares keeps the reference kernel's order: threads 0..255 run
// the strided per-thread chains (element t + 256 j, increasing j) and the
// two-level tree (eight 32-lane trees, then one over the 8 partials and 24
// zeros). The absmax (order-free) and the Q8 pack are spread over all NT
// threads, a K32 group per 32-lane half. sm is >= 18 floats of LDS. Ends
// with the block synchronised.
template <int NT>
__device__ __forceinline__ void rms_q8_row(const float* __restrict__ x, const uint16_t* __restrict__ gamma,
                                           float eps, int8_t* codes, float* scales, int32_t* sums,
                                           int* failure, float* sm, float* xs) {
  constexpr int kPer = kRmsHidden / 256, kGroups = kRmsHidden / 32, kHalves = NT / 32;
  constexpr int kSteps = kGroups / kHalves, kWaves = NT / 64;
  static_assert(kSteps * kHalves == kGroups && kWaves <= 16, "block shape");
  const uint32_t tid = threadIdx.x, lane32 = tid & 31u, half = tid >> 5;
  float xv[kSteps], gv[kSteps];
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {  // half h owns groups h + kHalves s
    const uint32_t i = (half + kHalves * st) * 32 + lane32;
    xv[st] = x[i];
    gv[st] = bf16_to_f32(gamma[i]);
  }
  float s = 0.f;
#pragma unroll
  for (int st = 0; st < kSteps; ++st) s = fmaxf(s, fabsf(xv[st]));
#pragma unroll
  for (int off = 32; off; off >>= 1) s = fmaxf(s, __shfl_xor(s, off));
  if ((tid & 63u) == 0) sm[tid >> 6] = s;
  __syncthreads();
  // every thread takes the block maximum itself (fmaxf is order-free)
  float scale = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) scale = fmaxf(scale, sm[w]);
  const float safe = scale == 0.f ? 1.f : scale;
  // Each thread divides its own elements once; the quotients go to LDS (xs,
  // kRmsHidden floats), where the sum of squares below reads them in the
  // reference's strided order, and stay in registers for the output.
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    xv[st] = xv[st] / safe;
    xs[(half + kHalves * st) * 32 + lane32] = xv[st];
  }
  __syncthreads();  // xs complete; every thread has read sm[0..kWaves)
  if (tid < 256) {
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const float q = xs[tid + 256 * j];
      sq = fmaf(q, q, sq);
    }
    sq = tree32_sum(sq);
    if (lane32 == 0) sm[tid >> 5] = sq;
  }
  __syncthreads();
  if (tid < 32) {
    float t = lane32 < 8 ? sm[lane32] : 0.f;
    t = tree32_sum(t);
    if (lane32 == 0) sm[17] = t;
  }
  __syncthreads();
  const float sumsq = sm[17];
  const float se = sqrtf(eps) / safe;
  const float inv = 1.0f / sqrtf(fmaf(se, se, sumsq / float(kRmsHidden)));
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    const float y = bf16_to_f32(f32_to_bf16_rne((1.0f + gv[st]) * (xv[st] * inv)));
    q8_group32(y, codes, scales, sums, half + kHalves * st, failure);
  }
  __syncthreads();
}

// Byte offsets of the 16-byte code word of (row, super-block kb, K32 group g)
// and of the 16-byte metadata row of (row, kb).
// 0x020D: tile row ((row/8)*kbs + kb)*8 + row%8; codes 128 B per tile row
//   (group g at g*16), metadata 16 B per tile row.
// 0x0240: chunk-major. Super-blocks are grouped in chunks of nk <= 8 (only the
//   last chunk is short); chunk c of all strips is contiguous, strip after
//   strip. Within (chunk, strip) the codes form eight planes of nk*128 B, one
//   per group, whose 16-byte entries are ordered (kb%8)*8 + row%8, and the
//   metadata is one such plane. One wave64 load instruction thus reads a whole
//   plane contiguously, and neighbouring waves (strips) read neighbouring
//   memory at the same time.
__host__ __device__ __forceinline__ uint64_t q4k_code_word(uint16_t layout, uint32_t row,
                                                          uint32_t kb, uint32_t g,
                                                          uint32_t kbs, uint32_t strips) {
  if (layout == QW38_LAYOUT_Q4K_CANDIDATE_V2)
    return ((uint64_t(row / 8) * kbs + kb) * 8 + row % 8) * 128 + g * 16;
  const uint32_t c = kb / 8, kq = kb % 8;
  const uint32_t nk = kbs - 8 * c < 8 ? kbs - 8 * c : 8;
  return uint64_t(strips) * 8192 * c + uint64_t(row / 8) * nk * 1024 + uint64_t(g) * nk * 128 +
         (kq * 8 + row % 8) * 16;
}
__host__ __device__ __forceinline__ uint64_t q4k_meta_row(uint16_t layout, uint32_t row,
                                                         uint32_t kb, uint32_t kbs,
                                                         uint32_t strips) {
  if (layout == QW38_LAYOUT_Q4K_CANDIDATE_V2)
    return ((uint64_t(row / 8) * kbs + kb) * 8 + row % 8) * 16;
  const uint32_t c = kb / 8, kq = kb % 8;
  const uint32_t nk = kbs - 8 * c < 8 ? kbs - 8 * c : 8;
  return uint64_t(strips) * 1024 * c + uint64_t(row / 8) * nk * 128 + (kq * 8 + row % 8) * 16;
}

// Fixed K segment of the Q6_K accumulation, in super-blocks (a function of K
// only, so every M, tiling and split sums the same segments in the same
// order): four segments from 16 super-blocks on, one below. The Q6_K MMQ and
// the Q6_K batched decode both accumulate each segment from zero and add the
// segment sums in ascending order.
__host__ __device__ constexpr uint32_t q6_seg_kb(uint32_t kbs) { return kbs >= 16 ? (kbs + 3) / 4 : kbs; }

// Library-owned device scratch (scratch.hip) for cross-block partial sums:
// the device address of this device's array for a launch on stream s, or
// null when `bytes` exceed it, another host thread holds it, or an earlier
// launch on another stream that used it has not completed (callers then take
// a path that needs no scratch and gives the same bits). A non-null result is
// handed back with scratch_release after the launches that use it.
// 64 MB: four Q6_K segment partials of a 5120-row weight up to M = 800.
constexpr uint64_t kScratchBytes = 64ull << 20;
void* scratch_acquire(hipStream_t s, uint64_t bytes, int* device);
void scratch_release(int device, hipStream_t s, bool launched);

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) once per (kernel, device)
// and size: the runtime call costs host time on every launch otherwise.
hipError_t set_max_lds(const void* kernel, int bytes);

// Ordered sum of Q6_K segment partials (segs arrays of m x n) + residual.
using Q6SegReduce = hipError_t (*)(const float* part, uint32_t segs, uint32_t m, uint32_t n,
                                   const float* residual, float* out, hipStream_t s);
uint64_t q6_mmq_dma_scratch_bytes(uint32_t mc, uint32_t n, uint32_t pk);
hipError_t launch_q6_mmq_dma(const WeightView& w, const Q8View& x, float* out, const float* residual,
                             hipStream_t s, void* scratch, int nw, int nj, uint32_t mc, Q6SegReduce reduce);

// ---- launchers (defined in the .hip files) ---------------------------------
hipError_t launch_pack_q8(const uint16_t* in, uint32_t m, uint32_t k, uint32_t pk,
                          int8_t* codes, float* scales, int32_t* sums, int* failure,
                          hipStream_t s);
// clear_failure (m = 1 only): the kernel zeroes *failure before it can set
// it, in place of a separate clearing launch.
hipError_t launch_rms_q8(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                         int8_t* codes, float* scales, int32_t* sums, int* failure,
                         hipStream_t s, bool clear_failure = false);
hipError_t launch_rms_bf16(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                           uint16_t* out, hipStream_t s);
hipError_t launch_swiglu_q8(const float* gate, const float* up, uint32_t m, uint32_t n,
                            int8_t* codes, float* scales, int32_t* sums, int* failure,
                            hipStream_t s);
// Compute units of the current device (cached per device).
int cu_count();
// FP8 (OCP E4M3FN) path.
hipError_t launch_pack_fp8(const uint16_t* x, uint32_t m, uint32_t k, uint8_t* codes, float* scales,
                           hipStream_t s);
hipError_t launch_fp8_gemv(const uint8_t* codes, const float* scales, uint32_t n, uint32_t k,
                           const uint16_t* x, void* y, const float* residual, int epilogue,
                           hipStream_t s);
// epilogue 0: raw FP32 [m][n]; otherwise a QW38_DECODE_* store of the first `valid` tokens.
hipError_t launch_fp8_gemm(const uint8_t* wc, const float* ws, uint32_t n, uint32_t k,
                           const uint8_t* xc, const float* xs, uint32_t m, void* y,
                           const float* residual, uint32_t valid, int epilogue, hipStream_t s);
hipError_t launch_fp8_store_bf16(const float* x, uint16_t* y, uint64_t count, hipStream_t s);
// NVFP4 (E2M1 + UE4M3 16-blocks, swizzled scales): activation pack (scales of
// pad128(m) rows), decode GEMV (paired when cb != nullptr) and the W4A4 GEMM
// (wsf: swizzled scales after the 256-byte header, wfactor: the header's FP32
// factor; epilogue 0 = raw FP32, a QW38_DECODE_* store, or
// QW38_DECODE_SWIGLU_BF16 with the gate projection FP32 [m][n] in residual).
// Fused RMS producers of hidden 5120: NVFP4 pack (codes [m][2560], swizzled
// scales of pad128(m) rows) and FP8 pack (codes [pm][5120], scales [40][pm],
// BF16 companion row when non-null).
hipError_t launch_rms_nvfp4(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                            uint8_t* codes, uint8_t* scales, hipStream_t s);
hipError_t launch_rms_fp8(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                          uint16_t* companion, uint8_t* codes, float* scales, hipStream_t s);
hipError_t launch_pack_nvfp4(const uint16_t* x, uint32_t m, uint32_t k, uint8_t* codes,
                             uint8_t* scales, hipStream_t s);
hipError_t launch_nvfp4_gemv(const uint8_t* ca, const uint8_t* sa, const uint8_t* cb,
                             const uint8_t* sb, uint32_t n, uint32_t pn, uint32_t k, uint32_t pk,
                             const uint16_t* x, void* ya, void* yb, const float* ra, const float* rb,
                             int epilogue, hipStream_t s);
hipError_t launch_nvfp4_gemm(const uint8_t* wc, const uint8_t* wsf, const float* wfactor,
                             uint32_t n, uint32_t code_rows, uint32_t pk, const uint8_t* xc,
                             const uint8_t* xs, uint32_t m, void* y, const float* residual,
                             int epilogue, hipStream_t s);
hipError_t launch_gemv(const WeightView& w, const Q8View& x, float* out,
                       const float* residual, hipStream_t s);
hipError_t launch_gemv_stream(const WeightView& w, const Q8View& x, float* out,
                              const float* residual, hipStream_t s, int ws_override,
                              uint32_t max_blocks);
// Q6_K (0x0241) streaming GEMV for M <= 2; hipErrorNotSupported otherwise.
hipError_t launch_q6k_stream(const WeightView& w, const Q8View& x, float* out,
                             const float* residual, hipStream_t s);
// Q4_K 0x020D at M = 2..8 on int8 MFMA; hipErrorNotSupported when the shape,
// alignment or LDS budget does not fit (the caller then uses the dot4 kernels).
hipError_t launch_q4k_mfma_decode(const WeightView& w, const Q8View& x, float* out,
                                  const float* residual, hipStream_t s);
// Q6_K 0x0241 at M = 3..8 on int8 MFMA; hipErrorNotSupported otherwise.
hipError_t launch_q6k_mfma_decode(const WeightView& w, const Q8View& x, float* out,
                                  const float* residual, hipStream_t s);
hipError_t launch_gemv_w64(const WeightView& w, const Q8View& x, float* out,
                           const float* residual, hipStream_t s);
hipError_t launch_mmq(const WeightView& w, const Q8View& x, float* out,
                      const float* residual, hipStream_t s);
// Fused gate + up MMQ (same geometry, Q4_K): one launch whose epilogue applies
// SwiGLU -> BF16 -> Q8 and writes the down projection's Q8 operand
// (codes [m][n], scales / sums [m][n / 32]) without FP32 gate / up slabs.
// Decode form of launch_mmq_glu (M = 1, layout 0x020D, n % 32 == 0): the
// streaming GEMV's arithmetic; hipErrorNotSupported where it does not apply.
bool gemv_glu_applies(const WeightView& gate, const WeightView& up, uint32_t m);
hipError_t launch_gemv_glu(const WeightView& gate, const WeightView& up, const Q8View& x, int8_t* codes,
                           float* scales, int32_t* sums, int* failure, hipStream_t s);
hipError_t launch_mmq_glu(const WeightView& gate, const WeightView& up, const Q8View& x,
                          int8_t* codes, float* scales, int32_t* sums, int* failure,
                          hipStream_t s);
hipError_t launch_prefill_bf16(const WeightView& a, const WeightView* b, const uint16_t* x,
                               uint32_t m, void* out, const float* residual, int epilogue,
                               hipStream_t s);
hipError_t launch_decode_bf16(const WeightView& a, const WeightView* b, const uint16_t* x,
                              void* out_a, void* out_b, const float* res_a, const float* res_b,
                              int epilogue, hipStream_t s);
// Q4G64 / Q8G32 / BF16 dense-tile decode_mmv layouts (same arguments).
hipError_t launch_decode_dense(const WeightView& a, const WeightView* b, const uint16_t* x,
                               void* out_a, void* out_b, const float* res_a, const float* res_b,
                               int epilogue, hipStream_t s);
hipError_t launch_group_dots(const WeightView& w, const Q8View& x, int32_t* dots,
                             hipStream_t s);
hipError_t launch_repack_q4k(const uint8_t* blocks, uint32_t n, uint32_t k, uint16_t layout,
                             uint8_t* codes, uint8_t* scales, hipStream_t s);
hipError_t launch_repack_q6k(const uint8_t* blocks, uint32_t n, uint32_t k, uint8_t* codes,
                             uint8_t* scales, hipStream_t s);
hipError_t launch_fill_zero_i32(int* p, uint32_t count, hipStream_t s);
hipError_t launch_quantize_q4k(const float* x, uint64_t blocks, uint8_t* out, int* failure,
                               hipStream_t s);
hipError_t launch_quantize_q6k(const float* x, uint64_t blocks, uint8_t* out, hipStream_t s);

}  // namespace qw38hip
