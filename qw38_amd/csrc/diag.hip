// Measurement aid: the shader clock under a full int8 matrix-core load.
//
// Every SIMD of every CU runs one wave issuing independent chains of
// v_mfma_i32_32x32x32_i8; wave 0 of block 0 records s_memtime (shader clock
// cycles) and s_memrealtime (constant 100 MHz) before and after its loop, so
// cycles / (realtime / 100 MHz) is the sclk the matrix cores actually ran at.
// The int8 dense peak at that clock is CUs x 8192 ops x sclk. The host also
// times the launch, which gives the achieved int8 rate of this pure-MFMA loop.
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

}  // namespace
}  // namespace qw38hip

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
