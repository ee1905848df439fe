// Measurement aid: the shader clock under a full int8 matrix-core load.
//
// Every SIMD of every CU runs one wave issuing independent chains of
// v_mfma_i32_32x32x32_i8; wave 0 of block 0 records s_memtime (shader clock
// cycles) and s_memrealtime (constant 100 MHz) before and after its loop, so
// cycles / (realtime / 100 MHz) is the sclk the matrix cores actually ran at.
// The int8 dense peak at that clock is CUs x 8192 ops x sclk. The host also
// times the launch, which gives the achieved int8 rate of this pure-MFMA loop.
//
// Second aid: a pure HBM read of a buffer (no arithmetic beyond an XOR fold
// that keeps the loads live), the ceiling a bandwidth-bound decode kernel of
// the same byte count is measured against. Mode 0 reads grid-stride (thread
// i of the grid reads 16 B at 16 (i + j grid_threads)); modes 1 and 2 give
// each wave one contiguous range and stream it 1 KB per load instruction,
// eight (mode 1) or sixteen (mode 2) loads in flight, the access pattern of
// the streaming GEMV.
//
// Third aid: how far FP32 VALU work and FP16 matrix-core work overlap on one
// SIMD (two waves per SIMD, eight per CU, register operands only): mode 0
// issues 16 independent v_mfma_f32_16x16x32_f16 per iteration, mode 1 64
// independent FP32 FMAs, mode 2 both interleaved one MFMA to four FMAs (the
// MMQ's per-group scale ratio), mode 3 eight MFMAs interleaved one to eight
// FMAs, mode 4 one MFMA-only and one FMA-only wave per SIMD (16 MFMAs, 64
// FMAs per SIMD and iteration). Time per iteration against the single-unit
// modes gives the overlap (the bench times the launches with events). Modes 5
// and 6 time 16 independent int8 MFMAs alone (16x16x32 and 16x16x64).
#include "common.hpp"

namespace qw38hip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_clock_kernel(uint32_t iters, uint64_t* ticks, int seed) {
  v4i a = {seed, seed + 1, seed + 2, seed + 3};
  v4i b = {seed ^ 5, seed ^ 6, seed ^ 7, seed ^ 9};
  v16i c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) c[j][i] = 0;
  const bool rec = blockIdx.x == 0 && threadIdx.x == 0;
  uint64_t t0 = 0, r0 = 0;
  if (rec) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[j], 0, 0, 0);
  }
  int acc = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc ^= c[j][i];
  if (rec) {
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    ticks[0] = t1 - t0;
    ticks[1] = r1 - r0;
  }
  if (acc == 0x7fffffff) ticks[2] = uint64_t(acc);  // keeps the chains live
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

template <int Mode>
__global__ __launch_bounds__(512, 1) void issue_probe_kernel(uint32_t iters, float s, uint64_t* ticks,
                                                             float* sink) {
  half8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = _Float16(float(threadIdx.x & 7u) + i);
    b[i] = _Float16(0.5f * i);
  }
  f4 acc[16];
  float x[64];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f4{0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 64; ++j) x[j] = float(threadIdx.x + j);
  const bool rec = blockIdx.x == 0 && threadIdx.x == 0;
  uint64_t t0 = 0;
  if (rec) t0 = __builtin_amdgcn_s_memtime();
  for (uint32_t it = 0; it < iters; ++it) {
    if constexpr (Mode == 0) {
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
    } else if constexpr (Mode == 1) {
#pragma unroll
      for (int j = 0; j < 64; ++j) x[j] = fmaf(x[j], s, 1.0f);
    } else if constexpr (Mode == 5 || Mode == 6) {  // int8 MFMAs alone: 16x16x32 / 16x16x64
      const v4i ia = {int(threadIdx.x), 3, 5, 7}, ib = {1, 2, 3, int(threadIdx.x)};
      const long la = long(threadIdx.x) * 77, lb = long(threadIdx.x) * 13 + 5;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        v4i c = __builtin_bit_cast(v4i, acc[j]);
        if constexpr (Mode == 5) c = __builtin_amdgcn_mfma_i32_16x16x32_i8(la, lb, c, 0, 0, 0);
        else c = __builtin_amdgcn_mfma_i32_16x16x64_i8(ia, ib, c, 0, 0, 0);
        acc[j] = __builtin_bit_cast(f4, c);
      }
    } else if constexpr (Mode == 4) {  // waves 0-3 MFMAs only, waves 4-7 FMAs only: one of each per SIMD
      if (threadIdx.x < 256) {
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
      } else {
#pragma unroll
        for (int j = 0; j < 64; ++j) x[j] = fmaf(x[j], s, 1.0f);
      }
    } else {
      constexpr int kM = Mode == 2 ? 16 : 8, kF = 64 / kM;
#pragma unroll
      for (int j = 0; j < kM; ++j) {
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
#pragma unroll
        for (int u = 0; u < kF; ++u) x[kF * j + u] = fmaf(x[kF * j + u], s, 1.0f);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, kF, 0);  // then kF VALU
      }
    }
  }
  if (rec) ticks[0] = __builtin_amdgcn_s_memtime() - t0;
  float r = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) r += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
#pragma unroll
  for (int j = 0; j < 64; ++j) r += x[j];
  if (r == 1234.5f) sink[0] = r;  // keeps the chains live
}

template <int Mode>
__global__ __launch_bounds__(256) void read_probe_kernel(const uint4* __restrict__ buf, uint64_t n16,
                                                         uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  if constexpr (Mode == 0) {
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    for (; i + 7 * stride < n16; i += 8 * stride) {
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = buf[i + u * stride];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
      const uint4 v = buf[i];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  } else {
    constexpr int U = Mode == 2 ? 16 : 8;  // 1 KB wave loads in flight
    const uint64_t waves = uint64_t(gridDim.x) * (blockDim.x / 64);
    const uint64_t wave = uint64_t(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64;
    const uint64_t chunks = n16 / 64;  // 1 KB wave loads
    const uint64_t c0 = chunks * wave / waves, c1 = chunks * (wave + 1) / waves;
    const uint32_t lane = threadIdx.x & 63u;
    uint64_t c = c0;
    for (; c + U <= c1; c += U) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (Mode == 3)  // non-temporal hint on the streamed lines
        {
          typedef uint32_t u4v __attribute__((ext_vector_type(4)));
          const u4v t = __builtin_nontemporal_load(reinterpret_cast<const u4v*>(&buf[(c + u) * 64 + lane]));
          v[u] = make_uint4(t.x, t.y, t.z, t.w);
        }
        else
          v[u] = buf[(c + u) * 64 + lane];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; c < c1; ++c) {
      const uint4 v = buf[c * 64 + lane];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;  // keeps the loads live; practically never stored
}

}  // namespace
}  // namespace qw38hip

extern "C" int qw38_read_probe(const void* buf, uint64_t bytes, uint32_t mode, uint32_t blocks_per_cu,
                               uint32_t* sink, uint64_t sink_len, void* stream) {
  using namespace qw38hip;
  if (buf == nullptr || sink == nullptr || bytes == 0 || bytes % 1024 || mode > 3 ||
      blocks_per_cu == 0 || blocks_per_cu > 32 || reinterpret_cast<uintptr_t>(buf) % 16)
    return QW38_INVALID_ARGUMENT;
  const uint32_t grid = uint32_t(cu_count()) * blocks_per_cu;
  if (sink_len < grid) return QW38_INVALID_ARGUMENT;
  auto kern = mode == 0   ? read_probe_kernel<0>
              : mode == 1 ? read_probe_kernel<1>
              : mode == 2 ? read_probe_kernel<2>
                          : read_probe_kernel<3>;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(buf), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? QW38_OK : QW38_STATUS;
}

extern "C" int qw38_mfma_clock_probe(uint32_t iterations, uint64_t* ticks, uint32_t* blocks,
                                     void* stream) {
  using namespace qw38hip;
  if (ticks == nullptr || blocks == nullptr || iterations == 0 || iterations > (1u << 24))
    return QW38_INVALID_ARGUMENT;
  const int cus = cu_count();
  *blocks = uint32_t(cus);  // 4 waves per block = one wave per SIMD
  hipLaunchKernelGGL(mfma_clock_kernel, dim3(cus), dim3(256), 0, static_cast<hipStream_t>(stream),
                     iterations, ticks, int(iterations & 0x7f));
  return hipGetLastError() == hipSuccess ? QW38_OK : QW38_STATUS;
}

extern "C" int qw38_issue_probe(uint32_t mode, uint32_t iterations, uint64_t* ticks, float* sink, void* stream) {
  using namespace qw38hip;
  if (ticks == nullptr || sink == nullptr || mode > 6 || iterations == 0 || iterations > (1u << 24))
    return QW38_INVALID_ARGUMENT;
  auto kern = mode == 0   ? issue_probe_kernel<0>
              : mode == 1 ? issue_probe_kernel<1>
              : mode == 2 ? issue_probe_kernel<2>
              : mode == 3 ? issue_probe_kernel<3>
              : mode == 4 ? issue_probe_kernel<4>
              : mode == 5 ? issue_probe_kernel<5>
                          : issue_probe_kernel<6>;
  hipLaunchKernelGGL(kern, dim3(cu_count()), dim3(512), 0, static_cast<hipStream_t>(stream), iterations, 0.999f,
                     ticks, sink);
  return hipGetLastError() == hipSuccess ? QW38_OK : QW38_STATUS;
}
