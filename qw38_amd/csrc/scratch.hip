// Library-owned device scratch for cross-block partial sums (the Q6_K MMQ
// split-K segments and the Q6_K batched decode's segment partials).
//
// The array is file-scope device memory: each GPU holds its own copy until
// the process ends. Host code only ever passes its device
// address, looked up with hipGetSymbolAddress once per device. A per-device
// record keeps calls on different streams apart: while an earlier launch on
// another stream that used the array has not completed, or another host
// thread holds it, scratch_acquire returns null and the caller takes its
// no-scratch path (the same bits, more time). Launches captured into a graph
// are not tracked: replays of such graphs on several streams at once must be
// serialized by the caller.
#include <mutex>
#include <tuple>
#include <vector>

#include "common.hpp"

namespace qw38hip {
namespace {

__device__ __align__(256) uint8_t device_scratch[kScratchBytes];

struct ScratchUse {
  void* ptr = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t stream = nullptr;
  bool recorded = false;
  bool busy = false;
  bool broken = false;
  uint64_t granted = 0, refused_size = 0, refused_busy = 0;  // qw38_scratch_stats
};
std::mutex g_mu;
ScratchUse g_use[64];

}  // namespace

void* scratch_acquire(hipStream_t s, uint64_t bytes, int* device) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  ScratchUse& u = g_use[dev];
  if (bytes > kScratchBytes) {
    ++u.refused_size;
    return nullptr;
  }
  if (u.broken || u.busy) {
    ++u.refused_busy;
    return nullptr;
  }
  if (!u.ptr) {
    if (hipGetSymbolAddress(&u.ptr, HIP_SYMBOL(device_scratch)) != hipSuccess ||
        hipEventCreateWithFlags(&u.done, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      u.ptr = nullptr;
      u.broken = true;
      return nullptr;
    }
  }
  if (u.recorded && u.stream != s) {
    if (hipEventQuery(u.done) != hipSuccess) {  // not ready (or failed): leave it alone
      (void)hipGetLastError();
      ++u.refused_busy;
      return nullptr;
    }
  }
  u.busy = true;
  ++u.granted;
  *device = dev;
  return u.ptr;
}

void scratch_release(int device, hipStream_t s, bool launched) {
  std::lock_guard<std::mutex> lock(g_mu);
  ScratchUse& u = g_use[device];
  u.busy = false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (launched && hipStreamIsCapturing(s, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone &&
      hipEventRecord(u.done, s) == hipSuccess) {
    u.recorded = true;
    u.stream = s;
  }
}

hipError_t set_max_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::vector<std::tuple<const void*, int, int>> done;  // (kernel, device, bytes)
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  for (auto const& d : done)
    if (std::get<0>(d) == kernel && std::get<1>(d) == dev && std::get<2>(d) >= bytes) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.emplace_back(kernel, dev, bytes);
  return e;
}

}  // namespace qw38hip

// Scratch requests on the current device since the process started:
// stats[0] granted, stats[1] refused for size (larger than the array),
// stats[2] refused because the array was in use (another thread, or earlier
// work on another stream). A refused request runs the no-scratch path.
extern "C" int qw38_scratch_stats(uint64_t* stats) {
  if (!stats) return QW38_INVALID_ARGUMENT;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return QW38_STATUS;
  }
  std::lock_guard<std::mutex> lock(qw38hip::g_mu);
  const qw38hip::ScratchUse& u = qw38hip::g_use[dev];
  stats[0] = u.granted;
  stats[1] = u.refused_size;
  stats[2] = u.refused_busy;
  return QW38_OK;
}
