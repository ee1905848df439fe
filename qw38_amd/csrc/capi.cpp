// C-ABI entry points: operand validation (all before any launch), dispatch to
// the gfx950 kernels, thread-local error reporting and allocation counters.
// Validation mirrors the reference's prelaunch contract: cuda/q4k_q8.cu:269-298
// (geometry, device residency, non-aliasing), cuda/prefill.cu:273-325.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <limits>
#include <mutex>

#include "common.hpp"
#include "profiling.hpp"

namespace {
using namespace qw38hip;

struct LastError {
  int status = QW38_OK;
  int hip_status = 0;
  char operation[96] = {0};
  char detail[256] = {0};
};
thread_local LastError g_err;

int fail(int status, const char* op, const char* detail, int hip_status = 0) {
  g_err.status = status;
  g_err.hip_status = hip_status;
  std::snprintf(g_err.operation, sizeof g_err.operation, "%s", op);
  std::snprintf(g_err.detail, sizeof g_err.detail, "%s", detail);
  return status;
}
int ok() {
  g_err = LastError{};
  return QW38_OK;
}
int hip_fail(hipError_t e, const char* op) {
  (void)hipGetLastError();  // consume the sticky error
  return fail(QW38_STATUS, op, hipGetErrorString(e), int(e));
}

std::atomic<uint64_t> g_mallocs{0}, g_frees{0}, g_live{0}, g_peak{0};

constexpr uint32_t pad_k(uint32_t k) { return k == 0 ? 0 : (k + 255u) / 256u * 256u; }
constexpr uint64_t pad_n(uint32_t n) { return n == 0 ? 0 : (uint64_t(n) + 7u) / 8u * 8u; }

// Activates the stream's device for the duration of a call (cuda/device.hpp:12-50).
struct DeviceScope {
  int previous = -1;
  bool restore = false;
  hipError_t status = hipSuccess;
  explicit DeviceScope(int device) {
    status = hipGetDevice(&previous);
    if (status == hipSuccess && previous != device) {
      status = hipSetDevice(device);
      restore = status == hipSuccess;
    }
  }
  ~DeviceScope() {
    if (restore) (void)hipSetDevice(previous);
  }
};

int stream_device(void* stream, int* device, const char* op) {
  hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), device)
                        : hipGetDevice(device);
  if (e != hipSuccess) return hip_fail(e, op);
  return QW38_OK;
}

struct Region {
  const void* p;
  uint64_t n;
  uint32_t alignment;
};

// Device-resident, aligned, inside one allocation (cuda/prefill.cu:273-309).
int validate_span(const Region& r, int device, const char* op) {
  if (r.n == 0) return QW38_OK;
  if (r.p == nullptr) return fail(QW38_INVALID_ARGUMENT, op, "null operand");
  const uintptr_t b = reinterpret_cast<uintptr_t>(r.p);
  if (r.alignment && b % r.alignment)
    return fail(QW38_INVALID_ARGUMENT, op, "misaligned operand");
  if (r.n > std::numeric_limits<uintptr_t>::max() - b)
    return fail(QW38_OVERFLOW, op, "address overflow");
  hipPointerAttribute_t attr{};
  hipError_t e = hipPointerGetAttributes(&attr, r.p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(QW38_INVALID_ARGUMENT, op, "operand is not device memory");
  }
  if (attr.type != hipMemoryTypeDevice || attr.device != device)
    return fail(QW38_INVALID_ARGUMENT, op, "operand is not memory of the stream's device");
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  e = hipMemGetAddressRange(&base, &size, const_cast<void*>(r.p));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(QW38_INVALID_ARGUMENT, op, "operand allocation range unknown");
  }
  const uintptr_t lo = reinterpret_cast<uintptr_t>(base);
  if (b < lo || b + r.n > lo + size)
    return fail(QW38_INVALID_ARGUMENT, op, "operand span exceeds its allocation");
  return QW38_OK;
}

int distinct(std::initializer_list<Region> regions, int device, const char* op) {
  const Region* rs = regions.begin();
  const size_t count = regions.size();
  for (size_t i = 0; i < count; ++i) {
    if (int st = validate_span(rs[i], device, op)) return st;
    if (rs[i].n == 0) continue;
    const uintptr_t b = reinterpret_cast<uintptr_t>(rs[i].p);
    for (size_t j = 0; j < i; ++j) {
      if (rs[j].n == 0) continue;
      const uintptr_t c = reinterpret_cast<uintptr_t>(rs[j].p);
      if (b < c + rs[j].n && c < b + rs[i].n)
        return fail(QW38_INVALID_ARGUMENT, "q8.alias", "live operands overlap");
    }
  }
  return QW38_OK;
}

bool valid_q8(const qw38_q8_input& x, uint32_t max_m) {
  return x.m && x.m <= max_m && x.k && x.k <= QW38_PROJECT_MAX_K && x.padded_k == pad_k(x.k) &&
         x.codes_len == uint64_t(x.m) * x.padded_k && x.scales_len == x.codes_len / 32 &&
         x.sums_len == x.scales_len;
}

bool layout_ok(uint16_t layout, uint16_t quantizer) {
  if (layout == QW38_LAYOUT_Q4K_CANDIDATE_V2 || layout == QW38_LAYOUT_Q4K_WAVE64)
    return quantizer == QW38_QUANTIZER_Q4K;
  if (layout == QW38_LAYOUT_Q6K_WAVE64) return quantizer == QW38_QUANTIZER_Q6K;
  return false;
}

int valid_weight(const qw38_weight& w, const char* op) {
  if (!w.n || w.n > QW38_PROJECT_MAX_N || !w.k || w.k > QW38_PROJECT_MAX_K ||
      !layout_ok(w.layout, w.quantizer) || w.padded_n != pad_n(w.n) ||
      w.padded_k != pad_k(w.k) ||
      w.codes_bytes != qw38_code_bytes(w.layout, w.padded_n, w.padded_k) ||
      w.scales_bytes != qw38_scale_bytes(w.layout, w.padded_n, w.padded_k))
    return fail(QW38_INVALID_ARGUMENT, op, "Q4_K/Q6_K geometry required");
  return QW38_OK;
}

uint32_t codes_alignment(const qw38_weight& w) {
  return w.layout == QW38_LAYOUT_Q4K_CANDIDATE_V2 ? 4u : 16u;
}
// 0x020D metadata may be only 2-byte aligned (the reference's fp16-backed span);
// the 0x0240 kernels load 16-byte metadata rows.
uint32_t scales_alignment(const qw38_weight& w) {
  return w.layout == QW38_LAYOUT_Q4K_WAVE64 ? 16u : 2u;
}

WeightView view(const qw38_weight& w) {
  return WeightView{static_cast<const uint8_t*>(w.codes), static_cast<const uint8_t*>(w.scales),
                    w.layout, w.n, w.k, w.padded_n, w.padded_k};
}

// ---- decode_mmv contract (cuda/decode_mmv.cu:245-560, restated) ----------
using DView = qw38_decode_view;
using DDesc = qw38_decode_desc;

bool reference_layout_quantizer(uint16_t layout, uint16_t quantizer) {
  switch (layout) {
    case QW38_DECODE_LAYOUT_FP8_V1: return quantizer == QW38_DECODE_QUANTIZER_FP8_V1;
    case QW38_DECODE_LAYOUT_NVFP4_V1: return quantizer == QW38_DECODE_QUANTIZER_NVFP4_V1;
    case QW38_LAYOUT_Q4K_CANDIDATE_V2: return quantizer == QW38_QUANTIZER_Q4K;
    case QW38_DECODE_LAYOUT_Q4G64_V0: return quantizer == QW38_DECODE_QUANTIZER_Q4G64_V0;
    case QW38_DECODE_LAYOUT_Q4G64_CANDIDATE_V1:
      return quantizer == QW38_DECODE_QUANTIZER_Q4G64_CANDIDATE_V1;
    case QW38_DECODE_LAYOUT_Q8G32_V0: return quantizer == QW38_DECODE_QUANTIZER_Q8G32_V0;
    case QW38_DECODE_LAYOUT_Q8G32_CANDIDATE_V1:
      return quantizer == QW38_DECODE_QUANTIZER_Q8G32_CANDIDATE_V1;
    case QW38_DECODE_LAYOUT_BF16_DENSE_TILE_V0: return quantizer == QW38_DECODE_QUANTIZER_NONE;
    default: return false;
  }
}

bool view_empty(const DView& v) {
  return v.pointer == nullptr && v.space == 0 && v.dtype == 0 && v.layout == 0 &&
         v.logical_n == 0 && v.logical_k == 0 && v.padded_n == 0 && v.padded_k == 0 &&
         v.bytes == 0 && v.alignment == 0 && v.writable == 0;
}

bool view_equal(const DView& a, const DView& b) {
  return a.pointer == b.pointer && a.space == b.space && a.dtype == b.dtype &&
         a.layout == b.layout && a.logical_n == b.logical_n && a.logical_k == b.logical_k &&
         a.padded_n == b.padded_n && a.padded_k == b.padded_k && a.bytes == b.bytes &&
         a.alignment == b.alignment && a.writable == b.writable;
}

int check_view(const DView& v, uint8_t dtype, uint16_t layout, uint32_t ln, uint32_t lk,
               uint32_t pn, uint32_t pk, uint64_t bytes, uint32_t min_align, bool writable,
               const char* op, const char* name) {
  const bool bad = v.pointer == nullptr || v.space != QW38_DECODE_SPACE_DEVICE ||
                   v.dtype != dtype || v.layout != layout || v.logical_n != ln ||
                   v.logical_k != lk || v.padded_n != pn || v.padded_k != pk ||
                   v.bytes != bytes || v.alignment < min_align ||
                   (v.alignment & (v.alignment - 1u)) != 0u ||
                   reinterpret_cast<uintptr_t>(v.pointer) % v.alignment != 0u ||
                   (v.writable != 0) != writable;
  if (!bad) return QW38_OK;
  char detail[128];
  std::snprintf(detail, sizeof detail, "%s typed view does not match the required contract", name);
  return fail(QW38_INVALID_ARGUMENT, op, detail);
}

bool views_overlap(const DView& a, const DView& b) {
  if (!a.pointer || !b.pointer || !a.bytes || !b.bytes) return false;
  const uintptr_t x = reinterpret_cast<uintptr_t>(a.pointer), y = reinterpret_cast<uintptr_t>(b.pointer);
  if (a.bytes > std::numeric_limits<uintptr_t>::max() - x ||
      b.bytes > std::numeric_limits<uintptr_t>::max() - y)
    return true;
  return x < y + b.bytes && y < x + a.bytes;
}

uint64_t decode_code_bytes_ref(uint16_t layout, uint32_t pn, uint32_t pk) {
  const uint64_t nk = uint64_t(pn) * pk;
  switch (layout) {
    case QW38_DECODE_LAYOUT_NVFP4_V1:
    case QW38_DECODE_LAYOUT_Q4G64_V0:
    case QW38_DECODE_LAYOUT_Q4G64_CANDIDATE_V1:
    case QW38_LAYOUT_Q4K_CANDIDATE_V2: return nk / 2;
    case QW38_DECODE_LAYOUT_FP8_V1:
    case QW38_DECODE_LAYOUT_Q8G32_V0:
    case QW38_DECODE_LAYOUT_Q8G32_CANDIDATE_V1: return nk;
    case QW38_DECODE_LAYOUT_BF16_DENSE_TILE_V0: return nk * 2;
    default: return 0;
  }
}

uint64_t decode_scale_bytes_ref(uint16_t layout, uint32_t pn, uint32_t pk) {
  const uint64_t rows = pn;
  switch (layout) {
    case QW38_DECODE_LAYOUT_NVFP4_V1: return 256 + (rows + 127) / 128 * 128 * (pk / 16u);
    case QW38_LAYOUT_Q4K_CANDIDATE_V2: return rows * (pk / 256u) * 16u;
    case QW38_DECODE_LAYOUT_Q4G64_V0:
    case QW38_DECODE_LAYOUT_Q4G64_CANDIDATE_V1: return rows * (pk / 64u) * 2u;
    case QW38_DECODE_LAYOUT_FP8_V1: return (rows / 128) * (pk / 128) * 4;
    case QW38_DECODE_LAYOUT_Q8G32_V0:
    case QW38_DECODE_LAYOUT_Q8G32_CANDIDATE_V1: return rows * (pk / 32u) * 2u;
    default: return 0;
  }
}

uint8_t decode_weight_dtype(uint16_t layout) {
  switch (layout) {
    case QW38_DECODE_LAYOUT_FP8_V1: return QW38_DECODE_DTYPE_FP8;
    case QW38_DECODE_LAYOUT_NVFP4_V1: return QW38_DECODE_DTYPE_NVFP4;
    case QW38_LAYOUT_Q4K_CANDIDATE_V2:
    case QW38_DECODE_LAYOUT_Q4G64_V0:
    case QW38_DECODE_LAYOUT_Q4G64_CANDIDATE_V1: return QW38_DECODE_DTYPE_Q4;
    case QW38_DECODE_LAYOUT_Q8G32_V0:
    case QW38_DECODE_LAYOUT_Q8G32_CANDIDATE_V1: return QW38_DECODE_DTYPE_Q8;
    default: return QW38_DECODE_DTYPE_BF16;
  }
}

uint32_t decode_group(uint16_t layout) {
  switch (layout) {
    case QW38_DECODE_LAYOUT_FP8_V1: return 128;
    case QW38_LAYOUT_Q4K_CANDIDATE_V2: return 256;
    case QW38_DECODE_LAYOUT_Q4G64_V0:
    case QW38_DECODE_LAYOUT_Q4G64_CANDIDATE_V1: return 64;
    case QW38_DECODE_LAYOUT_Q8G32_V0:
    case QW38_DECODE_LAYOUT_Q8G32_CANDIDATE_V1: return 32;
    default: return 1;
  }
}

// Geometry and typed views of one projection; paired_b allows the SwiGLU epilogue.
int decode_geometry(const DDesc& d, const char* op, bool paired_b) {
  if (!reference_layout_quantizer(d.layout, d.quantizer))
    return fail(QW38_INVALID_ARGUMENT, op, "layout/quantizer version mismatch");
  if (d.activation_policy != QW38_DECODE_ACTIVATION_BF16)
    return fail(QW38_INVALID_ARGUMENT, op, "unsupported decode activation policy");
  if (d.n == 0 || d.k == 0) return fail(QW38_INVALID_ARGUMENT, op, "N and K must be nonzero");
  if (d.layout == QW38_DECODE_LAYOUT_FP8_V1 && (d.n > 17408 || d.n % 128 || d.k % 256))
    return fail(QW38_INVALID_ARGUMENT, op, "FP8 requires aligned mixer geometry");
  if (d.layout == QW38_DECODE_LAYOUT_NVFP4_V1 && d.n > 248320)
    return fail(QW38_INVALID_ARGUMENT, op, "NVFP4 N exceeds model geometry");
  if (d.n > std::numeric_limits<uint32_t>::max() - 7u)
    return fail(QW38_OVERFLOW, op, "N exceeds the largest supported row-tile-padded value");
  if (d.k > QW38_DECODE_MAX_K || d.padded_k > QW38_DECODE_MAX_K)
    return fail(QW38_INVALID_ARGUMENT, op, "K exceeds decode staging limit 17408");
  if (d.padded_n != pad_n(d.n) || d.padded_k != pad_k(d.k))
    return fail(QW38_INVALID_ARGUMENT, op, "padded N/K metadata does not match layout tiles");
  if (d.layout == QW38_DECODE_LAYOUT_BF16_DENSE_TILE_V0) {
    if (d.n % 8 || d.k % 256)
      return fail(QW38_INVALID_ARGUMENT, op, "BF16 dense tile requires N%8==0 and K%256==0");
  } else if (d.k % decode_group(d.layout)) {
    return fail(QW38_INVALID_ARGUMENT, op, "logical K must divide the quantizer group");
  }
  const uint64_t want_codes = decode_code_bytes_ref(d.layout, d.padded_n, d.padded_k);
  const uint64_t want_scales = decode_scale_bytes_ref(d.layout, d.padded_n, d.padded_k);
  if (int st = check_view(d.codes, decode_weight_dtype(d.layout), d.layout, d.n, d.k, d.padded_n,
                          d.padded_k, want_codes, 16, false, op, "codes"))
    return st;
  if (want_scales == 0) {
    if (!view_empty(d.scales))
      return fail(QW38_INVALID_ARGUMENT, op, "BF16 dense tile must not supply scales");
  } else {
    const bool fp8 = d.layout == QW38_DECODE_LAYOUT_FP8_V1;
    const bool one_row = fp8 || d.layout == QW38_DECODE_LAYOUT_NVFP4_V1;
    const uint32_t rows = one_row ? 1u : d.padded_n;
    const uint32_t units = uint32_t(want_scales / rows / (fp8 ? 4u : 2u));
    if (int st = check_view(d.scales, fp8 ? QW38_DECODE_DTYPE_FP32 : QW38_DECODE_DTYPE_FP16,
                            d.layout, rows, units, rows, units, want_scales, one_row ? 16u : 2u,
                            false, op, "scales"))
      return st;
  }
  if (int st = check_view(d.input, QW38_DECODE_DTYPE_BF16, QW38_DECODE_LAYOUT_BF16_VECTOR_V0, d.k,
                          1, d.k, 1, uint64_t(d.k) * 2, 2, false, op, "input"))
    return st;
  if (d.epilogue < QW38_DECODE_STORE_BF16 || d.epilogue > QW38_DECODE_SWIGLU_BF16)
    return fail(QW38_INVALID_ARGUMENT, op, "unknown epilogue");
  if (d.epilogue == QW38_DECODE_SWIGLU_BF16 && !paired_b)
    return fail(QW38_INVALID_ARGUMENT, op, "SwiGLU epilogue requires paired gate/up launch");
  if (d.epilogue == QW38_DECODE_RESIDUAL_ADD_FP32) {
    const bool separate = !view_empty(d.output);
    if (int st = check_view(d.residual, QW38_DECODE_DTYPE_FP32, QW38_DECODE_LAYOUT_FP32_VECTOR_V0,
                            d.n, 1, d.n, 1, uint64_t(d.n) * 4, 4, !separate, op, "residual"))
      return st;
    if (separate) {
      if (int st = check_view(d.output, QW38_DECODE_DTYPE_FP32, QW38_DECODE_LAYOUT_FP32_VECTOR_V0,
                              d.n, 1, d.n, 1, uint64_t(d.n) * 4, 4, true, op, "output"))
        return st;
    }
  } else {
    if (!view_empty(d.residual))
      return fail(QW38_INVALID_ARGUMENT, op, "store epilogue must not supply residual");
    const bool f32 = d.epilogue == QW38_DECODE_STORE_FP32;
    if (int st = check_view(d.output, f32 ? QW38_DECODE_DTYPE_FP32 : QW38_DECODE_DTYPE_BF16,
                            f32 ? QW38_DECODE_LAYOUT_FP32_VECTOR_V0 : QW38_DECODE_LAYOUT_BF16_VECTOR_V0,
                            d.n, 1, d.n, 1, uint64_t(d.n) * (f32 ? 4 : 2), f32 ? 4u : 2u, true, op,
                            "output"))
      return st;
  }
  const DView* vs[] = {&d.codes, &d.scales, &d.input, &d.output, &d.residual};
  for (int i = 0; i < 5; ++i)
    for (int j = i + 1; j < 5; ++j)
      if (views_overlap(*vs[i], *vs[j]))
        return fail(QW38_INVALID_ARGUMENT, op, "operand views must not overlap");
  return QW38_OK;
}

// Layouts this build implements for decode (every layout the reference's
// decode_mmv accepts).
int decode_supported(const DDesc& d, const char* op) {
  switch (d.layout) {
    case QW38_DECODE_LAYOUT_FP8_V1:
    case QW38_DECODE_LAYOUT_NVFP4_V1:
    case QW38_LAYOUT_Q4K_CANDIDATE_V2:
    case QW38_DECODE_LAYOUT_Q4G64_V0:
    case QW38_DECODE_LAYOUT_Q4G64_CANDIDATE_V1:
    case QW38_DECODE_LAYOUT_Q8G32_V0:
    case QW38_DECODE_LAYOUT_Q8G32_CANDIDATE_V1:
    case QW38_DECODE_LAYOUT_BF16_DENSE_TILE_V0:
      return QW38_OK;
    default:
      return fail(QW38_INVALID_ARGUMENT, op, "decode layout not implemented on this build");
  }
}

int decode_paired_contract(const DDesc& a, const DDesc& b, const char* op) {
  if (int st = decode_geometry(a, op, true)) return st;
  DDesc bv = b;
  if (a.epilogue == QW38_DECODE_SWIGLU_BF16) {
    if (!view_empty(b.output) || !view_empty(b.residual))
      return fail(QW38_INVALID_ARGUMENT, op,
                  "SwiGLU paired B must not declare a separately materialized output");
    bv.output = a.output;
  }
  if (int st = decode_geometry(bv, op, true)) return st;
  if (b.layout != a.layout || b.quantizer != a.quantizer ||
      b.activation_policy != a.activation_policy || b.n != a.n || b.k != a.k ||
      b.padded_n != a.padded_n || b.padded_k != a.padded_k || b.epilogue != a.epilogue ||
      !view_equal(b.input, a.input))
    return fail(QW38_INVALID_ARGUMENT, op,
                "paired B must match A shape, layout, input, and epilogue contract");
  const DView* av[] = {&a.codes, &a.scales, &a.output, &a.residual};
  const DView* bw[] = {&b.codes, &b.scales, &b.output, &b.residual};
  for (const DView* x : av)
    for (const DView* y : bw)
      if (views_overlap(*x, *y))
        return fail(QW38_INVALID_ARGUMENT, op, "paired A/B operands must not overlap");
  return QW38_OK;
}

WeightView decode_weight(const DDesc& d) {
  return WeightView{static_cast<const uint8_t*>(d.codes.pointer),
                    static_cast<const uint8_t*>(d.scales.pointer), d.layout, d.n, d.k,
                    d.padded_n, d.padded_k};
}

int decode_launch(const DDesc& a, const DDesc* b, void* stream, const char* op) {
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  profiling::ScopedRange range(
      "qw38:op name=decode_mmv m=%u n=%u k=%u paired=%u layout=%u epilogue=%u compute=scalar_fp32", 1u,
      unsigned(a.n), unsigned(a.k), unsigned(b != nullptr), unsigned(a.layout), unsigned(a.epilogue));
  if (a.layout == QW38_DECODE_LAYOUT_FP8_V1) {  // cuda/fp8.cu:184-194
    if (b) return fail(QW38_INVALID_ARGUMENT, op, "FP8 paired SwiGLU is not supported");
    const hipError_t e = launch_fp8_gemv(
        static_cast<const uint8_t*>(a.codes.pointer), static_cast<const float*>(a.scales.pointer),
        a.n, a.k, static_cast<const uint16_t*>(a.input.pointer), a.output.pointer,
        static_cast<const float*>(a.residual.pointer), a.epilogue, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, op);
  }
  if (a.layout == QW38_DECODE_LAYOUT_NVFP4_V1) {  // cuda/decode_mmv.cu:94-102, 586-587
    const hipError_t e = launch_nvfp4_gemv(
        static_cast<const uint8_t*>(a.codes.pointer), static_cast<const uint8_t*>(a.scales.pointer),
        b ? static_cast<const uint8_t*>(b->codes.pointer) : nullptr,
        b ? static_cast<const uint8_t*>(b->scales.pointer) : nullptr, a.n, a.padded_n, a.k,
        a.padded_k, static_cast<const uint16_t*>(a.input.pointer), a.output.pointer,
        b ? b->output.pointer : nullptr, static_cast<const float*>(a.residual.pointer),
        b ? static_cast<const float*>(b->residual.pointer) : nullptr, a.epilogue,
        static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, op);
  }
  const WeightView wa = decode_weight(a);
  WeightView wb{};
  if (b) wb = decode_weight(*b);
  auto* launch = a.layout == QW38_LAYOUT_Q4K_CANDIDATE_V2 ? launch_decode_bf16 : launch_decode_dense;
  hipError_t e = launch(
      wa, b ? &wb : nullptr, static_cast<const uint16_t*>(a.input.pointer), a.output.pointer,
      b ? b->output.pointer : nullptr, static_cast<const float*>(a.residual.pointer),
      b ? static_cast<const float*>(b->residual.pointer) : nullptr, a.epilogue,
      static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

// ---- BF16 prefill contract (cuda/prefill.cu:434-466, 510-560, restated) ----
int prefill_weight(const qw38_weight& w, uint32_t tokens, const char* op) {
  if (!tokens || tokens > QW38_PROJECT_MAX_TOKENS || !w.codes || !w.n || !w.k ||
      w.k > QW38_PREFILL_MAX_K || w.padded_n != pad_n(w.n) || w.padded_k != pad_k(w.k) ||
      w.k % 256 || w.quantizer != QW38_QUANTIZER_Q4K ||
      (w.layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 && w.layout != QW38_LAYOUT_Q4K_WAVE64) ||
      w.codes_bytes != qw38_code_bytes(w.layout, w.padded_n, w.padded_k) ||
      w.scales_bytes != qw38_scale_bytes(w.layout, w.padded_n, w.padded_k) || !w.scales)
    return fail(QW38_INVALID_ARGUMENT, op, "weight, layout or token contract mismatch");
  if (w.layout != QW38_LAYOUT_Q4K_CANDIDATE_V2)
    return fail(QW38_INVALID_ARGUMENT, op, "prefill layout not implemented on this build");
  return QW38_OK;
}

hipError_t project(const qw38_weight& w, const Q8View& x, float* out, const float* residual,
                   hipStream_t s, const char* role = "projection") {
  profiling::ScopedRange range("qw38:op name=q4k_project m=%u n=%u k=%u role=%s residual=%u compute=%s",
                               unsigned(x.m), unsigned(w.n), unsigned(w.k), role,
                               unsigned(residual != nullptr), x.m <= 8 ? "integer_dot4_mfma" : "mfma_f16_exact");
  if (x.m <= 8) return launch_gemv(view(w), x, out, residual, s);
  return launch_mmq(view(w), x, out, residual, s);
}

// ---- FP8 projections (cuda/fp8.cu, restated validation) -----------------
struct FRegion {
  const void* p;
  uint64_t n;
  uint32_t alignment;
  bool write;
};

// Device-resident, aligned spans; a written span overlaps no other
// (cuda/fp8.cu:46-57).
int fp8_regions(std::initializer_list<FRegion> regions, int device) {
  const FRegion* rs = regions.begin();
  for (size_t i = 0; i < regions.size(); ++i) {
    if (int st = validate_span(Region{rs[i].p, rs[i].n, rs[i].alignment}, device, "fp8.v1")) return st;
    const uintptr_t a = reinterpret_cast<uintptr_t>(rs[i].p);
    for (size_t j = 0; j < i; ++j) {
      const uintptr_t b = reinterpret_cast<uintptr_t>(rs[j].p);
      if ((rs[i].write || rs[j].write) && a < b + rs[j].n && b < a + rs[i].n)
        return fail(QW38_INVALID_ARGUMENT, "fp8.v1", "invalid geometry, extent or alias");
    }
  }
  return QW38_OK;
}

int fp8_invalid() { return fail(QW38_INVALID_ARGUMENT, "fp8.v1", "invalid geometry, extent or alias"); }

bool fp8_geometry(const qw38_fp8_weight& w) {  // cuda/fp8.cu:58-61
  return w.n && w.n <= 17408 && w.k && w.k <= 17408 && !(w.n % 128) && !(w.k % 128) &&
         w.codes_len == uint64_t(w.n) * w.k && w.scales_len == uint64_t(w.n / 128) * (w.k / 128);
}

// ---- NVFP4 (cuda/nvfp4.cu, cuda/prefill.cu:218-221, 598-628, 680-715) ----
constexpr uint64_t pad128(uint64_t v) { return (v + 127) / 128 * 128; }
constexpr uint64_t align256(uint64_t v) { return (v + 255) / 256 * 256; }

// Engine-side NVFP4 scratch of `tokens` rows of K <= 5120: packed codes,
// swizzled scales, and the FP32 gate projection of the paired SwiGLU.
struct Nvfp4Scratch {
  uint64_t codes, scales, gate, bytes;
};
Nvfp4Scratch nvfp4_scratch(uint32_t tokens) {
  Nvfp4Scratch s{};
  s.codes = 0;
  s.scales = align256(pad128(tokens) * 2560);
  s.gate = s.scales + align256(pad128(tokens) * 320);
  s.bytes = s.gate + uint64_t(tokens) * 17408 * 4;
  return s;
}

// PrefillWeight contract of an NVFP4 weight (cuda/prefill.cu:218-221,
// 434-448): K <= 5120, K % 256 == 0, N <= 17408, N % 8 == 0, exact spans.
int nvfp4_weight(const qw38_weight& w, uint32_t tokens, const char* op) {
  if (!tokens || tokens > 1024 || !w.codes || !w.scales || w.layout != QW38_DECODE_LAYOUT_NVFP4_V1 ||
      w.quantizer != QW38_DECODE_QUANTIZER_NVFP4_V1 || !w.n || w.n > 17408 || w.n % 8 || !w.k ||
      w.k > 5120 || w.k % 256 || w.padded_n != pad_n(w.n) || w.padded_k != pad_k(w.k) ||
      w.codes_bytes != uint64_t(w.padded_n) * w.padded_k / 2 ||
      w.scales_bytes != 256 + pad128(w.padded_n) * (w.padded_k / 16))
    return fail(QW38_INVALID_ARGUMENT, op, "weight, layout or token contract mismatch");
  return QW38_OK;
}

hipError_t nvfp4_gemm(const qw38_weight& w, const uint8_t* xc, const uint8_t* xs, uint32_t tokens,
                      void* out, const float* residual, int epilogue, hipStream_t s) {
  const uint8_t* sc = static_cast<const uint8_t*>(w.scales);
  return launch_nvfp4_gemm(static_cast<const uint8_t*>(w.codes), sc + 256,
                           reinterpret_cast<const float*>(sc), w.n, w.padded_n, w.padded_k, xc, xs,
                           tokens, out, residual, epilogue, s);
}

}  // namespace

extern "C" {

int qw38_last_error(int* hip_status, char* operation, size_t operation_cap, char* detail,
                    size_t detail_cap) {
  if (hip_status) *hip_status = g_err.hip_status;
  if (operation && operation_cap) std::snprintf(operation, operation_cap, "%s", g_err.operation);
  if (detail && detail_cap) std::snprintf(detail, detail_cap, "%s", g_err.detail);
  return g_err.status;
}

void qw38_set_profiling(int enabled) { profiling::enabled = enabled != 0; }

uint64_t qw38_code_bytes(uint16_t layout, uint32_t padded_n, uint32_t padded_k) {
  const uint64_t nk = uint64_t(padded_n) * padded_k;
  switch (layout) {
    case QW38_LAYOUT_Q4K_CANDIDATE_V2:
    case QW38_LAYOUT_Q4K_WAVE64: return nk / 2;
    case QW38_LAYOUT_Q6K_WAVE64: return nk / 256 * 192;
    default: return 0;
  }
}

uint64_t qw38_scale_bytes(uint16_t layout, uint32_t padded_n, uint32_t padded_k) {
  const uint64_t blocks = uint64_t(padded_n) * (padded_k / 256);
  switch (layout) {
    case QW38_LAYOUT_Q4K_CANDIDATE_V2:
    case QW38_LAYOUT_Q4K_WAVE64: return blocks * 16;
    case QW38_LAYOUT_Q6K_WAVE64: return blocks * 18;
    default: return 0;
  }
}

int qw38_pack_q8(const uint16_t* input, uint64_t input_len, const qw38_q8_input* output,
                 int* failure, uint64_t failure_len, void* stream) {
  constexpr const char* op = "q8.pack";
  if (!output || !valid_q8(*output, QW38_PROJECT_MAX_TOKENS) ||
      input_len != uint64_t(output->m) * output->k || failure_len != 1)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  const qw38_q8_input& x = *output;
  if (int st = distinct({{input, input_len * 2, 2}, {x.codes, x.codes_len, 4},
                         {x.scales, x.scales_len * 4, 4}, {x.sums, x.sums_len * 4, 4},
                         {failure, 4, 4}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  profiling::ScopedRange range("qw38:op name=q8_pack m=%u n=%u k=%u", unsigned(x.m), unsigned(x.k), 1u);
  hipError_t e = launch_pack_q8(input, x.m, x.k, x.padded_k, x.codes, x.scales, x.sums, failure,
                                static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_q4k_q8_project(const qw38_weight* weight, const qw38_q8_input* input, float* output,
                        uint64_t output_len, const float* residual, uint64_t residual_len,
                        void* stream) {
  constexpr const char* op = "q8.project";
  if (!weight || !input) return fail(QW38_INVALID_ARGUMENT, op, "null descriptor");
  const qw38_weight& w = *weight;
  const qw38_q8_input& x = *input;
  if (int st = valid_weight(w, "q8.weight")) return st;
  if (!valid_q8(x, QW38_PROJECT_MAX_TOKENS) || x.k != w.k ||
      output_len != uint64_t(x.m) * w.n || (residual_len && residual_len != output_len) ||
      (residual_len == 0) != (residual == nullptr))
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{w.codes, w.codes_bytes, codes_alignment(w)},
                         {w.scales, w.scales_bytes, scales_alignment(w)},
                         {x.codes, x.codes_len, 4},
                         {x.scales, x.scales_len * 4, 4},
                         {x.sums, x.sums_len * 4, 4},
                         {output, output_len * 4, 4},
                         {residual, residual_len * 4, 4}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  const Q8View xv{x.codes, x.scales, x.sums, x.m, x.k, x.padded_k};
  hipError_t e = project(w, xv, output, residual, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "q4k_q8.project");
}

int qw38_q4k_q8_gate_up_swiglu(const qw38_weight* gate, const qw38_weight* up,
                               const qw38_q8_input* input, const qw38_q8_input* output,
                               int* failure, uint64_t failure_len, void* stream) {
  constexpr const char* op = "q8.gate_up";
  if (!gate || !up || !input || !output) return fail(QW38_INVALID_ARGUMENT, op, "null descriptor");
  const qw38_q8_input& x = *input;
  const qw38_q8_input& y = *output;
  for (const qw38_weight* w : {gate, up})
    if (int st = valid_weight(*w, "q8.weight")) return st;
  if (gate->layout == QW38_LAYOUT_Q6K_WAVE64 || gate->layout != up->layout)
    return fail(QW38_INVALID_ARGUMENT, "q8.weight", "gate/up must be Q4_K in one layout");
  if (!valid_q8(x, QW38_PROJECT_MAX_TOKENS) || !valid_q8(y, QW38_PROJECT_MAX_TOKENS) ||
      x.k != gate->k || up->k != gate->k || up->n != gate->n || gate->n % 32 != 0 ||
      gate->n != gate->padded_n || y.m != x.m || y.k != gate->n || y.padded_k != gate->n ||
      failure_len != 1 || !failure)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{gate->codes, gate->codes_bytes, codes_alignment(*gate)},
                         {gate->scales, gate->scales_bytes, scales_alignment(*gate)},
                         {up->codes, up->codes_bytes, codes_alignment(*up)},
                         {up->scales, up->scales_bytes, scales_alignment(*up)},
                         {x.codes, x.codes_len, 4},
                         {x.scales, x.scales_len * 4, 4},
                         {x.sums, x.sums_len * 4, 4},
                         {y.codes, y.codes_len, 4},
                         {y.scales, y.scales_len * 4, 4},
                         {y.sums, y.sums_len * 4, 4},
                         {failure, 4, 4}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  profiling::ScopedRange range("qw38:op name=q4k_gate_up_swiglu_q8 m=%u n=%u k=%u", unsigned(x.m),
                               unsigned(2 * gate->n), unsigned(gate->k));
  const Q8View xv{x.codes, x.scales, x.sums, x.m, x.k, x.padded_k};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = gemv_glu_applies(view(*gate), view(*up), x.m)
                     ? launch_gemv_glu(view(*gate), view(*up), xv, y.codes, y.scales, y.sums, failure, s)
                     : launch_mmq_glu(view(*gate), view(*up), xv, y.codes, y.scales, y.sums, failure, s);
  return e == hipSuccess ? ok() : hip_fail(e, "q4k_q8.gate_up");
}

uint64_t qw38_q8_mlp_workspace_bytes(uint32_t m) {
  return uint64_t(m) * (17408 + 17408 / 32 * 8 + 2 * 17408 * 4) + 4;
}

}  // extern "C"

namespace {
// Q8 MLP body shared by qw38_q4k_q8_mlp (caller workspace) and
// qw38_q4k_q8_mlp_static (the library's static scratch, own_workspace): the
// workspace of the static variant is private to the library, so it is left
// out of the caller-operand residency and aliasing checks.
int mlp_run(const qw38_weight* gate, const qw38_weight* up, const qw38_weight* down,
            const float* residual, const uint16_t* gamma, float eps, float* output, uint32_t m,
            void* workspace, uint64_t workspace_bytes, void* stream, int* submitted,
            int* pending_failure, bool own_workspace) {
  constexpr const char* op = "q8.mlp";
  if (submitted) *submitted = 0;
  if (!gate || !up || !down || !submitted) return fail(QW38_INVALID_ARGUMENT, op, "null descriptor");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!pending_failure) {
    // Public completion API rejects stream capture (cuda/graph.cpp:21-31).
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &cs);
    if (e != hipSuccess) return hip_fail(e, "graph.require_uncaptured");
    if (cs != hipStreamCaptureStatusNone)
      return fail(QW38_INVALID_ARGUMENT, "graph.require_uncaptured", "stream is capturing");
  }
  if (!m || m > QW38_Q8_MLP_MAX_TOKENS || workspace_bytes < qw38_q8_mlp_workspace_bytes(m) ||
      !std::isfinite(eps) || eps <= 0 || gate->n != 17408 || gate->k != 5120 ||
      up->n != gate->n || up->k != gate->k || down->n != 5120 || down->k != 17408)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  for (const qw38_weight* w : {gate, up, down})
    if (int st = valid_weight(*w, "q8.weight")) return st;
  if (gate->layout == QW38_LAYOUT_Q6K_WAVE64 || up->layout == QW38_LAYOUT_Q6K_WAVE64)
    return fail(QW38_INVALID_ARGUMENT, "q8.weight", "gate/up must be Q4_K");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{gate->codes, gate->codes_bytes, codes_alignment(*gate)},
                         {gate->scales, gate->scales_bytes, scales_alignment(*gate)},
                         {up->codes, up->codes_bytes, codes_alignment(*up)},
                         {up->scales, up->scales_bytes, scales_alignment(*up)},
                         {down->codes, down->codes_bytes, codes_alignment(*down)},
                         {down->scales, down->scales_bytes, scales_alignment(*down)},
                         {residual, uint64_t(m) * 5120 * 4, 4},
                         {gamma, 5120 * 2, 2},
                         {output, uint64_t(m) * 5120 * 4, 4},
                         {workspace, own_workspace ? 0 : workspace_bytes, 4},
                         {pending_failure, pending_failure ? 4u : 0u, 4}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  auto* codes = static_cast<int8_t*>(workspace);
  auto* scales = reinterpret_cast<float*>(codes + size_t(m) * 17408);
  auto* sums = reinterpret_cast<int32_t*>(scales + size_t(m) * 544);
  auto* g = reinterpret_cast<float*>(sums + size_t(m) * 544);
  auto* u = g + size_t(m) * 17408;
  int* flag = pending_failure ? pending_failure : reinterpret_cast<int*>(u + size_t(m) * 17408);
  // Prefill (m > 8) runs gate + up as one fused MMQ launch whose epilogue
  // writes the down operand's Q8 codes directly; its input operand then lives
  // in the (unused) gate slab so it does not alias the codes being written.
  // QW38_MLP_FUSED=0 selects the unfused chain (same bits; a tuning aid).
  static const bool fused_env = [] {
    const char* e = std::getenv("QW38_MLP_FUSED");
    return !(e && std::atoi(e) == 0);
  }();
  const bool fused = fused_env && gate->layout == up->layout &&
                     (m > 8 || gemv_glu_applies(view(*gate), view(*up), m));
  int8_t* in_codes = fused ? reinterpret_cast<int8_t*>(g) : codes;
  float* in_scales = fused ? reinterpret_cast<float*>(in_codes + size_t(m) * 5120) : scales;
  int32_t* in_sums = fused ? reinterpret_cast<int32_t*>(in_scales + size_t(m) * 160) : sums;
  *submitted = 1;
  auto bail = [&](hipError_t e, const char* what) {
    if (!pending_failure) (void)hipStreamSynchronize(s);
    return hip_fail(e, what);
  };
  hipError_t e = hipSuccess;
  // The internal flag is cleared on every call: at m = 1 by the RMS->Q8
  // launch itself (one block), otherwise by a fill kernel first.
  const bool clear_in_rms = !pending_failure && m == 1;
  if (!pending_failure && !clear_in_rms) {
    profiling::ScopedRange range("qw38:op name=q8_clear_failure bytes=4");
    if ((e = launch_fill_zero_i32(flag, 1, s)) != hipSuccess) return bail(e, "q8.clear_failure");
  }
  if ((e = launch_rms_q8(residual, gamma, eps, m, in_codes, in_scales, in_sums, flag, s, clear_in_rms)) !=
      hipSuccess)
    return bail(e, "q8.rms_pack");
  Q8View x{in_codes, in_scales, in_sums, m, 5120, 5120};
  if (fused) {
    profiling::ScopedRange range("qw38:op name=q4k_gate_up_swiglu_q8 m=%u n=%u k=%u", unsigned(m), 34816u,
                                 5120u);
    e = m > 8 ? launch_mmq_glu(view(*gate), view(*up), x, codes, scales, sums, flag, s)
              : launch_gemv_glu(view(*gate), view(*up), x, codes, scales, sums, flag, s);
    if (e != hipSuccess) return bail(e, "q4k_q8.gate_up");
  } else {
    if ((e = project(*gate, x, g, nullptr, s, "gate")) != hipSuccess) return bail(e, "q4k_q8.project");
    if ((e = project(*up, x, u, nullptr, s, "up")) != hipSuccess) return bail(e, "q4k_q8.project");
    profiling::ScopedRange range("qw38:op name=swiglu_q8_pack m=%u n=%u k=%u", unsigned(m), 17408u, 1u);
    if ((e = launch_swiglu_q8(g, u, m, 17408, codes, scales, sums, flag, s)) != hipSuccess)
      return bail(e, "q8.swiglu_pack");
  }
  x = Q8View{codes, scales, sums, m, 17408, 17408};
  if ((e = project(*down, x, output, residual, s, "down")) != hipSuccess)
    return bail(e, "q4k_q8.project");
  if (pending_failure) return ok();
  int bad = 0;
  {
    profiling::ScopedRange range("qw38:op name=q8_failure_readback bytes=4");
    if ((e = hipMemcpyAsync(&bad, flag, 4, hipMemcpyDeviceToHost, s)) != hipSuccess)
      return bail(e, "q8.failure");
  }
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream.sync");
  if (bad)
    return fail(QW38_INVALID_ARGUMENT, "q8.producer", "nonfinite producer or invalid Q8 scale");
  return ok();
}
}  // namespace

extern "C" {

int qw38_q4k_q8_mlp(const qw38_weight* gate, const qw38_weight* up, const qw38_weight* down,
                    const float* residual, const uint16_t* gamma, float eps, float* output,
                    uint32_t m, void* workspace, uint64_t workspace_bytes, void* stream,
                    int* submitted, int* pending_failure) {
  return mlp_run(gate, up, down, residual, gamma, eps, output, m, workspace, workspace_bytes,
                 stream, submitted, pending_failure, false);
}

}  // extern "C"

// ---- allocation-free Q8 MLP --------------------------------------------------
// The workspace of qw38_q4k_q8_mlp_static lives in this file-scope device array
// (each GPU holds its own copy, at its own address, until the process ends).
// In host code `scratch` only names the symbol: its device address on the
// current device comes from hipGetSymbolAddress, looked up once per device and
// kept in g_scratch_ptr; kernels and copies only ever see that address.
namespace {
constexpr uint32_t kStaticMlpMaxTokens = QW38_Q8_MLP_STATIC_MAX_TOKENS;
constexpr uint64_t kStaticMlpBytes =
    uint64_t(kStaticMlpMaxTokens) * (17408 + 17408 / 32 * 8 + 2 * 17408 * 4) + 4;
__device__ __align__(256) uint8_t scratch[kStaticMlpBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

// Per-device record of the last call that used the scratch: a call still
// running on the host (another thread) or a call whose device work was
// enqueued on another stream and has not completed makes a new call reject
// before any launch. `done` is created once per device at set-up and recorded
// after each uncaptured submission; calls on one stream are ordered by it.
struct StaticUse {
  hipEvent_t done = nullptr;
  hipStream_t stream = nullptr;
  bool recorded = false;
  bool busy = false;
};
StaticUse g_static_use[64];

// Device address of this device's scratch (device must be current).
int scratch_address(int device, void** out) {
  if (device < 0 || device >= 64) return fail(QW38_INVALID_ARGUMENT, "q8.mlp_static", "device index");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "q8.mlp_static.symbol");
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return QW38_OK;
}
}  // namespace

extern "C" {

uint64_t qw38_q8_mlp_static_scratch_bytes(void) { return kStaticMlpBytes; }

int qw38_q4k_q8_mlp_static(const qw38_weight* gate, const qw38_weight* up, const qw38_weight* down,
                           const float* residual, const uint16_t* gamma, float eps, float* output,
                           uint32_t m, void* stream, int* submitted, int* pending_failure) {
  constexpr const char* op = "q8.mlp_static";
  if (submitted) *submitted = 0;
  if (!submitted) return fail(QW38_INVALID_ARGUMENT, op, "null descriptor");
  if (m > kStaticMlpMaxTokens)
    return fail(QW38_INVALID_ARGUMENT, op,
                "m exceeds the static scratch capacity (QW38_Q8_MLP_STATIC_MAX_TOKENS = 64)");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  void* ws = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  StaticUse& use = g_static_use[device];
  {
    DeviceScope scope(device);
    if (scope.status != hipSuccess) return hip_fail(scope.status, op);
    if (int st = scratch_address(device, &ws)) return st;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!use.done) {
      hipError_t e = hipEventCreateWithFlags(&use.done, hipEventDisableTiming);
      if (e != hipSuccess) {
        use.done = nullptr;
        return hip_fail(e, "q8.mlp_static.event");
      }
    }
    if (use.busy)
      return fail(QW38_INVALID_ARGUMENT, op,
                  "the static scratch is in use by a concurrent call on this device");
    if (use.recorded && use.stream != s) {
      hipError_t q = hipEventQuery(use.done);
      if (q == hipErrorNotReady)
        return fail(QW38_INVALID_ARGUMENT, op,
                    "the static scratch is in use by unfinished work on another stream");
      if (q != hipSuccess) return hip_fail(q, "q8.mlp_static.event");
    }
    use.busy = true;
  }
  int st = mlp_run(gate, up, down, residual, gamma, eps, output, m, ws,
                   qw38_q8_mlp_workspace_bytes(m), stream, submitted, pending_failure, true);
  DeviceScope scope(device);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  use.busy = false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (*submitted && scope.status == hipSuccess && hipStreamIsCapturing(s, &cs) == hipSuccess &&
      cs == hipStreamCaptureStatusNone) {
    // Work left on the stream (a pending_failure call returns before it
    // completes) is what a call on another stream must wait for.
    if (hipEventRecord(use.done, s) == hipSuccess) {
      use.recorded = true;
      use.stream = s;
    }
  }
  return st;
}

int qw38_hidden_rms_q8(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                       int8_t* codes, float* scales, int32_t* sums, int* failure,
                       void* stream) {
  constexpr const char* op = "q8.rms";
  if (!m || m > QW38_PROJECT_MAX_TOKENS || !std::isfinite(eps) || eps <= 0)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid operands");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{residual, uint64_t(m) * 5120 * 4, 4}, {gamma, 5120 * 2, 2},
                         {codes, uint64_t(m) * 5120, 4}, {scales, uint64_t(m) * 160 * 4, 4},
                         {sums, uint64_t(m) * 160 * 4, 4}, {failure, 4, 4}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  hipError_t e = launch_rms_q8(residual, gamma, eps, m, codes, scales, sums, failure,
                               static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "q8.rms_pack");
}

int qw38_swiglu_q8(const float* gate, const float* up, uint32_t m, uint32_t n, int8_t* codes,
                   float* scales, int32_t* sums, int* failure, void* stream) {
  constexpr const char* op = "q8.swiglu";
  if (!m || !n || n % 256 || m > QW38_PROJECT_MAX_TOKENS || n > QW38_PROJECT_MAX_K)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  const uint64_t e_count = uint64_t(m) * n;
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{gate, e_count * 4, 4}, {up, e_count * 4, 4}, {codes, e_count, 4},
                         {scales, e_count / 32 * 4, 4}, {sums, e_count / 32 * 4, 4},
                         {failure, 4, 4}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  hipError_t e = launch_swiglu_q8(gate, up, m, n, codes, scales, sums, failure,
                                  static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "q8.swiglu_pack");
}

int qw38_q8_group_dots(const qw38_weight* weight, const qw38_q8_input* input, int32_t* dots,
                       uint64_t dots_len, void* stream) {
  constexpr const char* op = "q8.group_dots";
  if (!weight || !input) return fail(QW38_INVALID_ARGUMENT, op, "null descriptor");
  const qw38_weight& w = *weight;
  const qw38_q8_input& x = *input;
  if (int st = valid_weight(w, "q8.weight")) return st;
  if (!valid_q8(x, QW38_PROJECT_MAX_TOKENS) || x.k != w.k ||
      dots_len != uint64_t(x.m) * w.n * (w.padded_k / 32))
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{w.codes, w.codes_bytes, codes_alignment(w)},
                         {w.scales, w.scales_bytes, scales_alignment(w)}, {x.codes, x.codes_len, 4},
                         {dots, dots_len * 4, 4}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  const Q8View xv{x.codes, x.scales, x.sums, x.m, x.k, x.padded_k};
  hipError_t e = launch_group_dots(view(w), xv, dots, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

static int repack_common(const void* blocks, uint64_t blocks_bytes, uint64_t block_size,
                         uint32_t n, uint32_t k, uint16_t layout, void* codes,
                         uint64_t codes_bytes, void* scales, uint64_t scales_bytes,
                         void* stream, const char* op, int device) {
  if (!n || !k || k % 256 || k > QW38_PROJECT_MAX_K || n > QW38_PROJECT_MAX_N ||
      blocks_bytes != uint64_t(n) * (k / 256) * block_size ||
      codes_bytes != qw38_code_bytes(layout, uint32_t(pad_n(n)), k) ||
      scales_bytes != qw38_scale_bytes(layout, uint32_t(pad_n(n)), k))
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  return distinct({{blocks, blocks_bytes, 1}, {codes, codes_bytes, 16}, {scales, scales_bytes, 4}},
                  device, op);
}

int qw38_repack_q4k_blocks(const void* blocks, uint64_t blocks_bytes, uint32_t n, uint32_t k,
                           uint16_t layout, void* codes, uint64_t codes_bytes, void* scales,
                           uint64_t scales_bytes, void* stream) {
  constexpr const char* op = "upload.q4k";
  if (layout != QW38_LAYOUT_Q4K_CANDIDATE_V2 && layout != QW38_LAYOUT_Q4K_WAVE64)
    return fail(QW38_INVALID_ARGUMENT, op, "Q4_K layout required");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = repack_common(blocks, blocks_bytes, 144, n, k, layout, codes, codes_bytes, scales,
                             scales_bytes, stream, op, device))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = launch_fill_zero_i32(static_cast<int*>(codes), uint32_t(codes_bytes / 4), s);
  if (e == hipSuccess) e = launch_fill_zero_i32(static_cast<int*>(scales), uint32_t(scales_bytes / 4), s);
  if (e == hipSuccess)
    e = launch_repack_q4k(static_cast<const uint8_t*>(blocks), n, k, layout,
                          static_cast<uint8_t*>(codes), static_cast<uint8_t*>(scales), s);
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_repack_q6k_blocks(const void* blocks, uint64_t blocks_bytes, uint32_t n, uint32_t k,
                           void* codes, uint64_t codes_bytes, void* scales,
                           uint64_t scales_bytes, void* stream) {
  constexpr const char* op = "upload.q6k";
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = repack_common(blocks, blocks_bytes, 210, n, k, QW38_LAYOUT_Q6K_WAVE64, codes,
                             codes_bytes, scales, scales_bytes, stream, op, device))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = launch_fill_zero_i32(static_cast<int*>(codes), uint32_t(codes_bytes / 4), s);
  if (e == hipSuccess) e = launch_fill_zero_i32(static_cast<int*>(scales), uint32_t(scales_bytes / 4), s);
  if (e == hipSuccess)
    e = launch_repack_q6k(static_cast<const uint8_t*>(blocks), n, k, static_cast<uint8_t*>(codes),
                          static_cast<uint8_t*>(scales), s);
  return e == hipSuccess ? ok() : hip_fail(e, op);
}


int qw38_fp8_prepare(void* stream, int* sm_count) {
  constexpr const char* op = "fp8.prepare";
  if (!sm_count) return fail(QW38_INVALID_ARGUMENT, op, "null output");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  int v = 0;
  const hipError_t e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) return hip_fail(e, op);
  *sm_count = v;
  return ok();
}

int qw38_fp8_store_bf16(const float* x, uint16_t* y, uint64_t count, void* stream) {
  if (!count || count > 1024ull * 17408ull) return fp8_invalid();
  int device = 0;
  if (int st = stream_device(stream, &device, "fp8.store")) return st;
  if (int st = fp8_regions({{x, count * 4, 4, false}, {y, count * 2, 2, true}}, device)) return st;
  DeviceScope scope(device);
  const hipError_t e = launch_fp8_store_bf16(x, y, count, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "fp8.store");
}

int qw38_pack_fp8(const uint16_t* input, uint64_t input_len, uint32_t m, uint32_t k,
                  uint8_t* codes, uint64_t codes_len, float* scales, uint64_t scales_len,
                  void* stream) {
  if (!m || m > 1024 || !k || k > 17408 || input_len != uint64_t(m) * k)
    return fp8_invalid();
  const uint32_t pm = (m + 127) / 128 * 128, pk = (k + 127) / 128 * 128;
  if (codes_len != uint64_t(pm) * pk || scales_len != uint64_t(pm) * (pk / 128)) return fp8_invalid();
  int device = 0;
  if (int st = stream_device(stream, &device, "fp8.pack")) return st;
  if (int st = fp8_regions({{input, input_len * 2, 2, false}, {codes, codes_len, 16, true},
                            {scales, scales_len * 4, 16, true}}, device))
    return st;
  DeviceScope scope(device);
  const hipError_t e = launch_pack_fp8(input, m, k, codes, scales, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "fp8.pack");
}

int qw38_fp8_gemv(const qw38_fp8_weight* w, const uint16_t* x, uint64_t x_len, float* y,
                  uint64_t y_len, void* stream) {
  if (!w || !fp8_geometry(*w) || x_len != w->k || y_len != w->n) return fp8_invalid();
  int device = 0;
  if (int st = stream_device(stream, &device, "fp8.gemv")) return st;
  if (int st = fp8_regions({{w->codes, w->codes_len, 16, false}, {w->scales, w->scales_len * 4, 16, false},
                            {x, x_len * 2, 2, false}, {y, y_len * 4, 4, true}}, device))
    return st;
  DeviceScope scope(device);
  const hipError_t e = launch_fp8_gemv(w->codes, w->scales, w->n, w->k, x, y, nullptr,
                                       QW38_DECODE_STORE_FP32, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "fp8.gemv");
}

int qw38_fp8_gemm(const qw38_fp8_weight* w, const qw38_fp8_input* x, float* y, uint64_t y_len,
                  void* workspace, uint64_t workspace_bytes, int sm_count, void* stream) {
  if (!w || !x || !fp8_geometry(*w) || !x->m || x->m > 1024 || x->m % 128 || x->k != w->k ||
      x->codes_len != uint64_t(x->m) * x->k || x->scales_len != uint64_t(x->m) * (x->k / 128) ||
      y_len != uint64_t(x->m) * w->n || !workspace || !workspace_bytes || sm_count <= 0)
    return fp8_invalid();
  int device = 0;
  if (int st = stream_device(stream, &device, "fp8.gemm")) return st;
  if (int st = fp8_regions({{w->codes, w->codes_len, 16, false}, {w->scales, w->scales_len * 4, 16, false},
                            {x->codes, x->codes_len, 16, false}, {x->scales, x->scales_len * 4, 16, false},
                            {y, y_len * 4, 16, true}, {workspace, workspace_bytes, 256, true}},
                           device))
    return st;
  DeviceScope scope(device);
  const hipError_t e = launch_fp8_gemm(w->codes, w->scales, w->n, w->k, x->codes, x->scales, x->m, y,
                                       nullptr, x->m, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "fp8.gemm");
}

int qw38_fp8_project(const qw38_fp8_weight* w, const qw38_fp8_input* x, uint32_t tokens,
                     void* output, const float* residual, int epilogue, void* stream) {
  // PrefillEngine::project FP8 branch (cuda/prefill.cu:218-219, 565-593)
  const bool res = epilogue == QW38_DECODE_RESIDUAL_ADD_FP32;
  if (!w || !x || !fp8_geometry(*w) || w->n > 12288 || w->k > 6144 || w->k % 256 || !tokens ||
      tokens > 1024 || x->m != (tokens + 127) / 128 * 128 || x->k != w->k ||
      x->codes_len != uint64_t(x->m) * x->k || x->scales_len != uint64_t(x->m) * (x->k / 128))
    return fp8_invalid();
  if (epilogue < QW38_DECODE_STORE_BF16 || epilogue > QW38_DECODE_RESIDUAL_ADD_FP32 ||
      res != (residual != nullptr) || !output)
    return fail(QW38_INVALID_ARGUMENT, "prefill.project",
                "input, output, position or epilogue contract mismatch");
  int device = 0;
  if (int st = stream_device(stream, &device, "fp8.project")) return st;
  const uint64_t cells = uint64_t(tokens) * w->n;
  const uint32_t ob = epilogue == QW38_DECODE_STORE_BF16 ? 2 : 4;
  if (int st = fp8_regions({{w->codes, w->codes_len, 16, false}, {w->scales, w->scales_len * 4, 16, false},
                            {x->codes, x->codes_len, 16, false}, {x->scales, x->scales_len * 4, 16, false},
                            {residual, res ? cells * 4 : 0, 16, false},
                            {output, cells * ob, ob == 2 ? 8u : 16u, true}},
                           device))
    return st;
  DeviceScope scope(device);
  const hipError_t e = launch_fp8_gemm(w->codes, w->scales, w->n, w->k, x->codes, x->scales, x->m,
                                       output, residual, tokens, epilogue,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, "fp8.project");
}

int qw38_pack_nvfp4(const uint16_t* input, uint32_t m, uint32_t k, uint8_t* codes,
                    uint64_t codes_bytes, uint8_t* scales, uint64_t scales_bytes, void* stream) {
  constexpr const char* op = "nvfp4.pack";  // cuda/nvfp4.cu:72-82
  if (!input || !codes || !scales || !m || m > 1024 || !k || k > 17408)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid operands");
  const uint64_t pk = pad_k(k);
  if (codes_bytes < uint64_t(m) * pk / 2 || scales_bytes < pad128(m) * (pk / 16))
    return fail(QW38_INVALID_ARGUMENT, op, "invalid operands");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = fp8_regions({{input, uint64_t(m) * k * 2, 2, false}, {codes, uint64_t(m) * pk / 2, 8, true},
                            {scales, pad128(m) * (pk / 16), 1, true}}, device))
    return st;
  DeviceScope scope(device);
  const hipError_t e = launch_pack_nvfp4(input, m, k, codes, scales, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_hidden_rms_nvfp4(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                          uint8_t* codes, uint8_t* scales, void* stream) {
  constexpr const char* op = "nvfp4.rms";  // cuda/activation.cu:507-520
  if (!residual || !gamma || !codes || !scales || !m || m > 1024 || !std::isfinite(eps) || eps <= 0.f)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid operands");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = fp8_regions({{residual, uint64_t(m) * 5120 * 4, 4, false}, {gamma, 5120 * 2, 2, false},
                            {codes, uint64_t(m) * 2560, 8, true}, {scales, pad128(m) * 320, 1, true}},
                           device))
    return st;
  DeviceScope scope(device);
  const hipError_t e = launch_rms_nvfp4(residual, gamma, eps, m, codes, scales, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_hidden_rms_fp8(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                        uint16_t* companion, uint8_t* codes, float* scales, void* stream) {
  constexpr const char* op = "fp8.rms";  // cuda/activation.cu:522-534
  if (!residual || !gamma || !codes || !scales || !m || m > 1024 || !std::isfinite(eps) || eps <= 0.f)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid operands");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  const uint64_t pm = pad128(m);
  if (int st = fp8_regions({{residual, uint64_t(m) * 5120 * 4, 4, false}, {gamma, 5120 * 2, 2, false},
                            {codes, pm * 5120, 16, true}, {scales, pm * 40 * 4, 4, true},
                            {companion, companion ? uint64_t(m) * 5120 * 2 : 0, 2, true}},
                           device))
    return st;
  DeviceScope scope(device);
  const hipError_t e = launch_rms_fp8(residual, gamma, eps, m, companion, codes, scales,
                                      static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_nvfp4_gemm_tile(const void* codes, const void* scales, const uint8_t* activation,
                         const uint8_t* activation_scales, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t row_start, float* output, void* stream) {
  constexpr const char* op = "nvfp4.gemm";  // cuda/nvfp4.cu:83-116
  if (!codes || !scales || !activation || !activation_scales || !output || !m || m > 1024 || !n ||
      n > 17408 || n % 8 || !k || k > 5120 || k % 256 || row_start % 128)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid tile");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  const uint8_t* wc = static_cast<const uint8_t*>(codes) + uint64_t(row_start) * k / 2;
  const uint8_t* sc = static_cast<const uint8_t*>(scales);
  const uint8_t* wsf = sc + 256 + uint64_t(row_start) * (k / 16);
  if (int st = fp8_regions({{wc, uint64_t(n) * k / 2, 16, false}, {sc, 4, 4, false},
                            {wsf, pad128(n) * (k / 16), 16, false},
                            {activation, uint64_t(m) * k / 2, 16, false},
                            {activation_scales, pad128(m) * (k / 16), 16, false},
                            {output, uint64_t(m) * n * 4, 16, true}},
                           device))
    return st;
  DeviceScope scope(device);
  const hipError_t e = launch_nvfp4_gemm(wc, wsf, reinterpret_cast<const float*>(sc), n, n, k, activation,
                                         activation_scales, m, output, nullptr, 0,
                                         static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

uint64_t qw38_nvfp4_workspace_bytes(uint32_t tokens) { return nvfp4_scratch(tokens).bytes; }

int qw38_nvfp4_project(const qw38_weight* weight, const uint16_t* input, uint32_t tokens,
                       void* output, const float* residual, int epilogue, void* workspace,
                       uint64_t workspace_bytes, void* stream) {
  constexpr const char* op = "prefill.project";  // cuda/prefill.cu:598-628
  if (!weight) return fail(QW38_INVALID_ARGUMENT, op, "null weight");
  const qw38_weight& w = *weight;
  if (int st = nvfp4_weight(w, tokens, "prefill.weight")) return st;
  const bool res = epilogue == QW38_DECODE_RESIDUAL_ADD_FP32;
  if (!input || !output || res != (residual != nullptr) ||
      (epilogue != QW38_DECODE_STORE_BF16 && epilogue != QW38_DECODE_STORE_FP32 && !res))
    return fail(QW38_INVALID_ARGUMENT, op, "input, output, position or epilogue contract mismatch");
  const Nvfp4Scratch ws = nvfp4_scratch(tokens);
  if (!workspace || workspace_bytes < ws.gate)
    return fail(QW38_INVALID_ARGUMENT, op, "workspace too small");
  const uint32_t ob = epilogue == QW38_DECODE_STORE_BF16 ? 2u : 4u;
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{w.codes, w.codes_bytes, 16}, {w.scales, w.scales_bytes, 16},
                         {input, uint64_t(tokens) * w.k * 2, 2},
                         {output, uint64_t(tokens) * w.n * ob, ob == 2 ? 8u : 16u},
                         {residual, res ? uint64_t(tokens) * w.n * 4 : 0, 16},
                         {workspace, ws.gate, 256}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* base = static_cast<uint8_t*>(workspace);
  hipError_t e = launch_pack_nvfp4(input, tokens, w.k, base + ws.codes, base + ws.scales, s);
  if (e == hipSuccess)
    e = nvfp4_gemm(w, base + ws.codes, base + ws.scales, tokens, output, residual, epilogue, s);
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_nvfp4_paired_swiglu(const qw38_weight* gate, const qw38_weight* up,
                             const uint16_t* normalized, uint16_t* swiglu, uint32_t tokens,
                             void* workspace, uint64_t workspace_bytes, void* stream) {
  constexpr const char* op = "prefill.swiglu";  // cuda/prefill.cu:680-715
  if (!gate || !up) return fail(QW38_INVALID_ARGUMENT, op, "null weight");
  if (int st = nvfp4_weight(*gate, tokens, "prefill.weight")) return st;
  if (int st = nvfp4_weight(*up, tokens, "prefill.weight")) return st;
  if (!normalized || !swiglu || gate->n != up->n || gate->k != up->k)
    return fail(QW38_INVALID_ARGUMENT, op, "paired weight or activation contract mismatch");
  const Nvfp4Scratch ws = nvfp4_scratch(tokens);
  if (!workspace || workspace_bytes < ws.bytes)
    return fail(QW38_INVALID_ARGUMENT, op, "workspace too small");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{gate->codes, gate->codes_bytes, 16}, {gate->scales, gate->scales_bytes, 16},
                         {up->codes, up->codes_bytes, 16}, {up->scales, up->scales_bytes, 16},
                         {normalized, uint64_t(tokens) * gate->k * 2, 2},
                         {swiglu, uint64_t(tokens) * gate->n * 2, 8}, {workspace, ws.bytes, 256}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* base = static_cast<uint8_t*>(workspace);
  float* g = reinterpret_cast<float*>(base + ws.gate);
  hipError_t e = launch_pack_nvfp4(normalized, tokens, gate->k, base + ws.codes, base + ws.scales, s);
  if (e == hipSuccess) e = nvfp4_gemm(*gate, base + ws.codes, base + ws.scales, tokens, g, nullptr, 0, s);
  if (e == hipSuccess)
    e = nvfp4_gemm(*up, base + ws.codes, base + ws.scales, tokens, swiglu, g, QW38_DECODE_SWIGLU_BF16, s);
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_decode_mmv(const qw38_decode_desc* desc, void* stream) {
  constexpr const char* op = "decode_mmv";
  if (!desc) return fail(QW38_INVALID_ARGUMENT, op, "null descriptor");
  if (int st = decode_geometry(*desc, op, false)) return st;
  if (int st = decode_supported(*desc, op)) return st;
  return decode_launch(*desc, nullptr, stream, op);
}

int qw38_decode_mmv_paired(const qw38_decode_desc* a, const qw38_decode_desc* b, void* stream) {
  constexpr const char* op = "decode_mmv_paired";
  if (!a || !b) return fail(QW38_INVALID_ARGUMENT, op, "null descriptor");
  if (int st = decode_paired_contract(*a, *b, op)) return st;
  if (int st = decode_supported(*a, op)) return st;
  return decode_launch(*a, b, stream, op);
}

int qw38_decode_ab_bf16(const qw38_decode_desc* a, const qw38_decode_desc* b, void* stream) {
  constexpr const char* op = "decode_ab_bf16";
  if (!a || !b) return fail(QW38_INVALID_ARGUMENT, op, "null descriptor");
  if (a->layout != QW38_DECODE_LAYOUT_BF16_DENSE_TILE_V0 || a->quantizer != QW38_DECODE_QUANTIZER_NONE)
    return fail(QW38_INVALID_ARGUMENT, op, "a/b contraction requires cuda_bf16_dense_tile_v0");
  if (a->epilogue != QW38_DECODE_STORE_FP32)
    return fail(QW38_INVALID_ARGUMENT, op, "a/b contraction requires FP32 output");
  if (int st = decode_paired_contract(*a, *b, op)) return st;
  return decode_launch(*a, b, stream, op);
}

int qw38_decode_mmv_ranges(const qw38_decode_desc* ranges, uint32_t count, void* stream) {
  constexpr const char* op = "decode_mmv_ranges";
  if (!ranges || count < 2 || count > 3)
    return fail(QW38_INVALID_ARGUMENT, op, "ranged launch requires two or three projections");
  const DDesc& first = ranges[0];
  if (first.layout == QW38_DECODE_LAYOUT_NVFP4_V1)
    return fail(QW38_INVALID_ARGUMENT, op,
                "NVFP4 supports single or paired gate/up launches only");
  if (first.epilogue != QW38_DECODE_STORE_BF16)
    return fail(QW38_INVALID_ARGUMENT, op, "ranged projections store BF16");
  if (int st = decode_geometry(first, "decode_mmv_ranges[0]", false)) return st;
  for (uint32_t i = 1; i < count; ++i) {
    const DDesc& d = ranges[i];
    if (d.layout != first.layout || d.quantizer != first.quantizer ||
        d.activation_policy != first.activation_policy)
      return fail(QW38_INVALID_ARGUMENT, op, "ranged projections must share one layout family");
    if (d.k != first.k || d.padded_k != first.padded_k)
      return fail(QW38_INVALID_ARGUMENT, op, "ranged projections must share K");
    if (!view_equal(d.input, first.input))
      return fail(QW38_INVALID_ARGUMENT, op, "ranged projections must share the input");
    if (d.epilogue != QW38_DECODE_STORE_BF16)
      return fail(QW38_INVALID_ARGUMENT, op, "ranged projections store BF16");
    if (int st = decode_geometry(d, op, false)) return st;
  }
  for (uint32_t i = 0; i < count; ++i)
    for (uint32_t j = i + 1; j < count; ++j) {
      const DView* l[] = {&ranges[i].codes, &ranges[i].scales, &ranges[i].output};
      const DView* r[] = {&ranges[j].codes, &ranges[j].scales, &ranges[j].output};
      for (const DView* x : l)
        for (const DView* y : r)
          if (views_overlap(*x, *y))
            return fail(QW38_INVALID_ARGUMENT, op, "ranged projection operand spans must not overlap");
    }
  if (int st = decode_supported(first, op)) return st;
  // One launch per range on the same stream: same results as one fused grid.
  for (uint32_t i = 0; i < count; ++i)
    if (int st = decode_launch(ranges[i], nullptr, stream, op)) return st;
  return ok();
}

int qw38_prefill_project(const qw38_weight* weight, const uint16_t* input, uint32_t tokens,
                         void* output, const float* residual, int epilogue, void* stream) {
  constexpr const char* op = "prefill.project";
  if (!weight) return fail(QW38_INVALID_ARGUMENT, op, "null weight");
  const qw38_weight& w = *weight;
  if (int st = prefill_weight(w, tokens, "prefill.weight")) return st;
  const bool res = epilogue == QW38_DECODE_RESIDUAL_ADD_FP32;
  if (!input || !output || res != (residual != nullptr) ||
      (epilogue != QW38_DECODE_STORE_BF16 && epilogue != QW38_DECODE_STORE_FP32 && !res))
    return fail(QW38_INVALID_ARGUMENT, op, "input, output, position or epilogue contract mismatch");
  const uint32_t ob = epilogue == QW38_DECODE_STORE_BF16 ? 2u : 4u;
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{w.codes, w.codes_bytes, 2},
                         {w.scales, w.scales_bytes, 2},
                         {input, uint64_t(tokens) * w.k * 2, 2},
                         {output, uint64_t(tokens) * w.n * ob, ob},
                         {residual, res ? uint64_t(tokens) * w.n * 4 : 0, 4}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  hipError_t e = launch_prefill_bf16(view(w), nullptr, input, tokens, output, residual, epilogue,
                                     static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_prefill_paired_swiglu(const qw38_weight* gate, const qw38_weight* up,
                               const uint16_t* normalized, uint16_t* swiglu, uint32_t tokens,
                               void* stream) {
  constexpr const char* op = "prefill.swiglu";
  if (!gate || !up) return fail(QW38_INVALID_ARGUMENT, op, "null weight");
  if (int st = prefill_weight(*gate, tokens, "prefill.weight")) return st;
  if (int st = prefill_weight(*up, tokens, "prefill.weight")) return st;
  if (!normalized || !swiglu || gate->n != up->n || gate->k != up->k ||
      gate->layout != up->layout || gate->quantizer != up->quantizer)
    return fail(QW38_INVALID_ARGUMENT, op, "paired weight or activation contract mismatch");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{gate->codes, gate->codes_bytes, 2},
                         {gate->scales, gate->scales_bytes, 2},
                         {up->codes, up->codes_bytes, 2},
                         {up->scales, up->scales_bytes, 2},
                         {normalized, uint64_t(tokens) * gate->k * 2, 2},
                         {swiglu, uint64_t(tokens) * gate->n * 2, 2}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  const WeightView u = view(*up);
  hipError_t e = launch_prefill_bf16(view(*gate), &u, normalized, tokens, swiglu, nullptr,
                                     QW38_DECODE_STORE_BF16, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_hidden_rms_bf16(const float* residual, const uint16_t* gamma, float eps, uint32_t m,
                         uint16_t* output, void* stream) {
  constexpr const char* op = "hidden_rms";
  if (!residual || !gamma || !output) return fail(QW38_INVALID_ARGUMENT, op, "null residual, gamma, or out");
  if (!m || m > QW38_PROJECT_MAX_TOKENS || !std::isfinite(eps) || eps <= 0.f)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid token count or epsilon");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{residual, uint64_t(m) * 5120 * 4, 4}, {gamma, 5120 * 2, 2},
                         {output, uint64_t(m) * 5120 * 2, 2}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  hipError_t e = launch_rms_bf16(residual, gamma, eps, m, output, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

uint64_t qw38_prefill_mlp_workspace_bytes(uint32_t tokens) {
  return align256(uint64_t(tokens) * (5120u * 2u + 17408u * 2u)) + nvfp4_scratch(tokens).bytes;
}

int qw38_prefill_mlp(const qw38_weight* gate, const qw38_weight* up, const qw38_weight* down,
                     const float* h_mid, const uint16_t* gamma, float eps, float* next_h,
                     uint32_t tokens, void* workspace, uint64_t workspace_bytes, void* stream) {
  constexpr const char* op = "prefill.mlp";
  if (!gate || !up || !down || !h_mid || !gamma || !next_h || !workspace ||
      !std::isfinite(eps) || eps <= 0.f || gate->n != 17408 || gate->k != 5120 ||
      down->n != 5120 || down->k != 17408 || up->n != gate->n || up->k != gate->k ||
      up->layout != gate->layout || up->quantizer != gate->quantizer ||
      workspace_bytes < qw38_prefill_mlp_workspace_bytes(tokens))
    return fail(QW38_INVALID_ARGUMENT, op, "MLP shape or pointer contract mismatch");
  // NVFP4 gate/up run the fused RMS->NVFP4 producer and the W4A4 pair
  // (cuda/prefill.cu:766-772); the down projection (K = 17408) stays Q4_K.
  const bool nv = gate->layout == QW38_DECODE_LAYOUT_NVFP4_V1;
  for (const qw38_weight* w : {gate, up})
    if (int st = nv ? nvfp4_weight(*w, tokens, "prefill.weight") : prefill_weight(*w, tokens, "prefill.weight"))
      return st;
  if (int st = prefill_weight(*down, tokens, "prefill.weight")) return st;
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  const uint64_t act = uint64_t(tokens) * 5120;
  if (int st = distinct({{h_mid, act * 4, 4}, {next_h, act * 4, 4}, {gamma, 5120 * 2, 2},
                         {workspace, qw38_prefill_mlp_workspace_bytes(tokens), 2},
                         {gate->codes, gate->codes_bytes, 2}, {gate->scales, gate->scales_bytes, 2},
                         {up->codes, up->codes_bytes, 2}, {up->scales, up->scales_bytes, 2},
                         {down->codes, down->codes_bytes, 2}, {down->scales, down->scales_bytes, 2}},
                        device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* normalized = static_cast<uint16_t*>(workspace);
  uint16_t* sw = normalized + act;
  hipError_t e = hipSuccess;
  if (nv) {
    uint8_t* nb = static_cast<uint8_t*>(workspace) + align256(uint64_t(tokens) * (5120u * 2u + 17408u * 2u));
    const Nvfp4Scratch ws = nvfp4_scratch(tokens);
    float* g = reinterpret_cast<float*>(nb + ws.gate);
    e = launch_rms_nvfp4(h_mid, gamma, eps, tokens, nb + ws.codes, nb + ws.scales, s);
    if (e == hipSuccess) e = nvfp4_gemm(*gate, nb + ws.codes, nb + ws.scales, tokens, g, nullptr, 0, s);
    if (e == hipSuccess)
      e = nvfp4_gemm(*up, nb + ws.codes, nb + ws.scales, tokens, sw, g, QW38_DECODE_SWIGLU_BF16, s);
  } else {
    e = launch_rms_bf16(h_mid, gamma, eps, tokens, normalized, s);
    const WeightView u = view(*up);
    if (e == hipSuccess)
      e = launch_prefill_bf16(view(*gate), &u, normalized, tokens, sw, nullptr,
                              QW38_DECODE_STORE_BF16, s);
  }
  if (e == hipSuccess)
    e = launch_prefill_bf16(view(*down), nullptr, sw, tokens, next_h, h_mid,
                            QW38_DECODE_RESIDUAL_ADD_FP32, s);
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_quantize_q4k_blocks(const float* x, uint64_t x_len, uint32_t n, uint32_t k,
                             void* blocks, uint64_t blocks_bytes, int* failure, void* stream) {
  constexpr const char* op = "quantize.q4k";
  if (!n || !k || k % 256 || x_len != uint64_t(n) * k ||
      blocks_bytes != uint64_t(n) * (k / 256) * 144)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{x, x_len * 4, 4}, {blocks, blocks_bytes, 4}, {failure, 4, 4}}, device, op))
    return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  hipError_t e = launch_quantize_q4k(x, uint64_t(n) * (k / 256), static_cast<uint8_t*>(blocks),
                                     failure, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_quantize_q6k_blocks(const float* x, uint64_t x_len, uint32_t n, uint32_t k,
                             void* blocks, uint64_t blocks_bytes, void* stream) {
  constexpr const char* op = "quantize.q6k";
  if (!n || !k || k % 256 || x_len != uint64_t(n) * k ||
      blocks_bytes != uint64_t(n) * (k / 256) * 210)
    return fail(QW38_INVALID_ARGUMENT, op, "invalid geometry");
  int device = 0;
  if (int st = stream_device(stream, &device, op)) return st;
  if (int st = distinct({{x, x_len * 4, 4}, {blocks, blocks_bytes, 2}}, device, op)) return st;
  DeviceScope scope(device);
  if (scope.status != hipSuccess) return hip_fail(scope.status, op);
  hipError_t e = launch_quantize_q6k(x, uint64_t(n) * (k / 256), static_cast<uint8_t*>(blocks),
                                     static_cast<hipStream_t>(stream));
  return e == hipSuccess ? ok() : hip_fail(e, op);
}

int qw38_device_malloc(void** pointer, uint64_t bytes) {
  if (!pointer || !bytes) return fail(QW38_INVALID_ARGUMENT, "device.malloc", "empty allocation");
  hipError_t e = hipMalloc(pointer, bytes);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  g_mallocs.fetch_add(1);
  const uint64_t live = g_live.fetch_add(bytes) + bytes;
  uint64_t peak = g_peak.load();
  while (live > peak && !g_peak.compare_exchange_weak(peak, live)) {
  }
  return ok();
}

int qw38_device_free(void* pointer, uint64_t bytes) {
  if (!pointer) return ok();
  hipError_t e = hipFree(pointer);
  g_frees.fetch_add(1);
  g_live.fetch_sub(std::min<uint64_t>(bytes, g_live.load()));
  return e == hipSuccess ? ok() : hip_fail(e, "hipFree");
}

uint64_t qw38_malloc_count(void) { return g_mallocs.load(); }
uint64_t qw38_free_count(void) { return g_frees.load(); }
uint64_t qw38_live_bytes(void) { return g_live.load(); }
uint64_t qw38_peak_live_bytes(void) { return g_peak.load(); }

void qw38_record_malloc(uint64_t bytes) {
  g_mallocs.fetch_add(1);
  const uint64_t live = g_live.fetch_add(bytes) + bytes;
  uint64_t peak = g_peak.load();
  while (live > peak && !g_peak.compare_exchange_weak(peak, live)) {
  }
}

void qw38_record_free(uint64_t bytes) {
  g_frees.fetch_add(1);
  g_live.fetch_sub(std::min<uint64_t>(bytes, g_live.load()));
}

}  // extern "C"
