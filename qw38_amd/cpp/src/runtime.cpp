// qw38::cuda runtime pieces on HIP: errors, device/stream/event/graph
// handles, device buffers with the library's allocation counters, copies and
// uploads (interfaces of cuda/{error,stream,event,graph,alloc,buffer,copy,
// upload}.hpp in Enucatl/qw38).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <string>
#include <utility>

#include "cuda/alloc.hpp"
#include "cuda/buffer.hpp"
#include "cuda/copy.hpp"
#include "cuda/error.hpp"
#include "cuda/event.hpp"
#include "cuda/graph.hpp"
#include "cuda/prefill.hpp"
#include "cuda/stream.hpp"
#include "cuda/upload.hpp"
#include "qw38_hip.h"

namespace qw38::cuda {

// ---- errors -----------------------------------------------------------------
char const* code_name(ErrorCode code) noexcept {
  switch (code) {
    case ErrorCode::Status: return "Status";
    case ErrorCode::InvalidArgument: return "InvalidArgument";
    case ErrorCode::Overflow: return "Overflow";
  }
  return "Unknown";
}

Error from_status(hipError_t status, std::string_view operation, std::source_location loc) {
  std::string detail = hipGetErrorString(status);
  detail += " at ";
  detail += loc.file_name();
  detail += ":" + std::to_string(loc.line());
  return Error{ErrorCode::Status, static_cast<int>(status), std::string(operation), detail};
}

Error make_error(ErrorCode code, std::string_view operation, std::string_view detail) {
  return Error{code, static_cast<int>(hipSuccess), std::string(operation), std::string(detail)};
}

std::string error_message(Error const& error) {
  std::string s = code_name(error.code);
  s += " in " + error.operation + ": " + error.detail;
  if (error.cuda_status != 0) s += " (hip " + std::to_string(error.cuda_status) + ")";
  return s;
}

expected<void, Error> from_abi(int status) {
  if (status == QW38_OK) return {};
  int hip = 0;
  char op[96] = {0};
  char detail[256] = {0};
  const int code = qw38_last_error(&hip, op, sizeof op, detail, sizeof detail);
  const ErrorCode c = code == QW38_OVERFLOW          ? ErrorCode::Overflow
                      : code == QW38_INVALID_ARGUMENT ? ErrorCode::InvalidArgument
                                                      : ErrorCode::Status;
  return unexpected(Error{c, hip, op, detail});
}

// ---- stream -------------------------------------------------------------------
namespace {
std::atomic<bool> g_fail_next_sync{false};
std::atomic<std::uint64_t> g_sync_count{0};
std::atomic<bool> g_fail_next_instantiate{false};
}  // namespace

namespace testing {
void fail_next_stream_sync() noexcept { g_fail_next_sync.store(true); }
std::uint64_t stream_sync_count() noexcept { return g_sync_count.load(); }
void fail_next_graph_instantiation() noexcept { g_fail_next_instantiate.store(true); }
}  // namespace testing

Stream::Stream(Stream&& other) noexcept
    : stream_(std::exchange(other.stream_, nullptr)), device_(std::exchange(other.device_, -1)) {}

Stream& Stream::operator=(Stream&& other) noexcept {
  if (this != &other) {
    (void)destroy();
    stream_ = std::exchange(other.stream_, nullptr);
    device_ = std::exchange(other.device_, -1);
  }
  return *this;
}

Stream::~Stream() { (void)destroy(); }

hipError_t Stream::destroy() noexcept {
  if (!stream_) return hipSuccess;
  hipError_t e = hipStreamDestroy(stream_);
  stream_ = nullptr;
  return e;
}

expected<Stream, Error> Stream::create() {
  int device = 0;
  if (auto st = check(hipGetDevice(&device), "hipGetDevice"); !st)
    return unexpected(st.error());
  hipStream_t s = nullptr;
  // default priority: streams of different priorities are not used here
  if (auto st = check(hipStreamCreateWithFlags(&s, hipStreamDefault), "hipStreamCreate"); !st)
    return unexpected(st.error());
  return Stream(s, device);
}

expected<void, Error> Stream::close() {
  auto guard = activate();
  if (!guard) {
    (void)destroy();
    return unexpected(guard.error());
  }
  return check(destroy(), "hipStreamDestroy");
}

expected<DeviceGuard, Error> Stream::activate() const {
  if (empty()) return unexpected(make_error(ErrorCode::InvalidArgument, "stream", "empty stream"));
  return DeviceGuard::activate(device_, "hipSetDevice");
}

expected<void, Error> Stream::sync() const {
  auto guard = activate();
  if (!guard) return unexpected(guard.error());
  if (auto st = check(hipStreamSynchronize(stream_), "hipStreamSynchronize"); !st) return st;
  g_sync_count.fetch_add(1);
  if (g_fail_next_sync.exchange(false))
    return unexpected(make_error(ErrorCode::Status, "hipStreamSynchronize",
                                      "injected synchronization failure"));
  return {};
}

// ---- events -------------------------------------------------------------------
Event::Event(Event&& other) noexcept
    : event_(std::exchange(other.event_, nullptr)), device_(std::exchange(other.device_, -1)) {}

Event& Event::operator=(Event&& other) noexcept {
  if (this != &other) {
    (void)destroy();
    event_ = std::exchange(other.event_, nullptr);
    device_ = std::exchange(other.device_, -1);
  }
  return *this;
}

Event::~Event() { (void)destroy(); }

hipError_t Event::destroy() noexcept {
  if (!event_) return hipSuccess;
  hipError_t e = hipEventDestroy(event_);
  event_ = nullptr;
  return e;
}

expected<Event, Error> Event::create() {
  int device = 0;
  if (auto st = check(hipGetDevice(&device), "hipGetDevice"); !st)
    return unexpected(st.error());
  hipEvent_t e = nullptr;
  if (auto st = check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate"); !st)
    return unexpected(st.error());
  return Event(e, device);
}

expected<Event, Error> Event::create_timing() {
  int device = 0;
  if (auto st = check(hipGetDevice(&device), "hipGetDevice"); !st)
    return unexpected(st.error());
  hipEvent_t e = nullptr;
  if (auto st = check(hipEventCreateWithFlags(&e, hipEventDefault), "hipEventCreate"); !st)
    return unexpected(st.error());
  return Event(e, device);
}

expected<void, Error> Event::close() { return check(destroy(), "hipEventDestroy"); }

expected<void, Error> Event::record(Stream const& stream) const {
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return check(hipEventRecord(event_, stream.native()), "hipEventRecord");
}

expected<void, Error> Event::wait(Stream const& stream) const {
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return check(hipStreamWaitEvent(stream.native(), event_, 0), "hipStreamWaitEvent");
}

expected<void, Error> Event::sync() const {
  return check(hipEventSynchronize(event_), "hipEventSynchronize");
}

expected<float, Error> elapsed_ms(Event const& start, Event const& end) {
  float ms = 0.f;
  if (auto st = check(hipEventElapsedTime(&ms, start.native(), end.native()), "hipEventElapsedTime");
      !st)
    return unexpected(st.error());
  return ms;
}

// ---- graphs -------------------------------------------------------------------
expected<void, Error> require_uncaptured(Stream const& stream) {
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  hipStreamCaptureStatus status{};
  if (auto st = check(hipStreamIsCapturing(stream.native(), &status), "hipStreamIsCapturing"); !st)
    return st;
  if (status != hipStreamCaptureStatusNone)
    return unexpected(make_error(ErrorCode::InvalidArgument, "stream.capture",
                                      "public completion API does not support capture"));
  return {};
}

Graph::~Graph() {
  if (capturing_) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(stream_, &g);
    if (g) (void)hipGraphDestroy(g);
  }
  if (exec_) (void)hipGraphExecDestroy(exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
}

expected<Graph, Error> Graph::begin(Stream const& stream) {
  if (auto st = require_uncaptured(stream); !st) return unexpected(st.error());
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  if (auto st = check(hipStreamBeginCapture(stream.native(), hipStreamCaptureModeThreadLocal),
                      "hipStreamBeginCapture");
      !st)
    return unexpected(st.error());
  Graph g;
  g.stream_ = stream.native();
  g.device_ = stream.device();
  g.capturing_ = true;
  return g;
}

expected<void, Error> Graph::finish() {
  if (!capturing_)
    return unexpected(make_error(ErrorCode::InvalidArgument, "graph.finish", "not capturing"));
  auto guard = DeviceGuard::activate(device_, "hipSetDevice");
  if (!guard) return unexpected(guard.error());
  capturing_ = false;
  if (auto st = check(hipStreamEndCapture(stream_, &graph_), "hipStreamEndCapture"); !st) return st;
  if (g_fail_next_instantiate.exchange(false))
    return unexpected(make_error(ErrorCode::Status, "hipGraphInstantiate",
                                      "injected instantiation failure"));
  return check(hipGraphInstantiate(&exec_, graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
}

expected<void, Error> Graph::launch(Stream const& stream) const {
  if (!exec_)
    return unexpected(make_error(ErrorCode::InvalidArgument, "graph.launch", "empty graph"));
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return check(hipGraphLaunch(exec_, stream.native()), "hipGraphLaunch");
}

// ---- allocation counters --------------------------------------------------------
std::uint64_t malloc_count() noexcept { return qw38_malloc_count(); }
std::uint64_t free_count() noexcept { return qw38_free_count(); }
std::uint64_t live_bytes() noexcept { return qw38_live_bytes(); }
std::uint64_t peak_live_bytes() noexcept { return qw38_peak_live_bytes(); }
void record_malloc(std::uint64_t bytes) noexcept { qw38_record_malloc(bytes); }
void record_free(std::uint64_t bytes) noexcept { qw38_record_free(bytes); }

// ---- device buffers ---------------------------------------------------------------
DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept
    : ptr_(std::exchange(other.ptr_, nullptr)),
      bytes_(std::exchange(other.bytes_, 0)),
      device_(std::exchange(other.device_, -1)) {}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
  if (this != &other) {
    (void)destroy();
    ptr_ = std::exchange(other.ptr_, nullptr);
    bytes_ = std::exchange(other.bytes_, 0);
    device_ = std::exchange(other.device_, -1);
  }
  return *this;
}

DeviceBuffer::~DeviceBuffer() { (void)destroy(); }

hipError_t DeviceBuffer::destroy() noexcept {
  if (!ptr_) return hipSuccess;
  int previous = 0;
  const bool switch_device = hipGetDevice(&previous) == hipSuccess && previous != device_;
  if (switch_device) (void)hipSetDevice(device_);
  const int st = qw38_device_free(ptr_, bytes_);
  if (switch_device) (void)hipSetDevice(previous);
  ptr_ = nullptr;
  bytes_ = 0;
  return st == QW38_OK ? hipSuccess : hipErrorInvalidValue;
}

expected<DeviceBuffer, Error> DeviceBuffer::allocate(std::uint64_t bytes) {
  int device = 0;
  if (auto st = check(hipGetDevice(&device), "hipGetDevice"); !st)
    return unexpected(st.error());
  return allocate(bytes, device);
}

expected<DeviceBuffer, Error> DeviceBuffer::allocate(std::uint64_t bytes, int device) {
  if (bytes == 0)
    return unexpected(make_error(ErrorCode::InvalidArgument, "device.allocate", "empty allocation"));
  auto guard = DeviceGuard::activate(device, "hipSetDevice");
  if (!guard) return unexpected(guard.error());
  void* p = nullptr;
  if (auto st = from_abi(qw38_device_malloc(&p, bytes)); !st) return unexpected(st.error());
  return DeviceBuffer(p, bytes, device);
}

expected<void, Error> DeviceBuffer::close() {
  return check(destroy(), "hipFree");
}

namespace {
// Fill kernels: stream-ordered and safe to capture (no memset nodes).
__global__ void fill_bytes_kernel(std::uint8_t* p, std::uint64_t n, std::uint8_t seed, bool ramp) {
  for (std::uint64_t i = blockIdx.x * std::uint64_t(blockDim.x) + threadIdx.x; i < n;
       i += std::uint64_t(gridDim.x) * blockDim.x)
    p[i] = ramp ? std::uint8_t(seed + i) : seed;
}

expected<void, Error> fill(void* ptr, std::uint64_t bytes, std::uint8_t seed, bool ramp,
                                Stream const& stream, char const* op) {
  if (!ptr && bytes) return unexpected(make_error(ErrorCode::InvalidArgument, op, "null pointer"));
  if (!bytes) return {};
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const std::uint64_t blocks = std::min<std::uint64_t>((bytes + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_bytes_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream.native(),
                     static_cast<std::uint8_t*>(ptr), bytes, seed, ramp);
  return check(hipGetLastError(), op);
}
}  // namespace

expected<void, Error> zero(DeviceBuffer& buffer, Stream const& stream) {
  return fill(buffer.data(), buffer.bytes(), 0, false, stream, "zero");
}

expected<void, Error> zero(void* ptr, std::uint64_t bytes, Stream const& stream) {
  return fill(ptr, bytes, 0, false, stream, "zero");
}

expected<void, Error> fill_pattern(void* dst, std::uint64_t bytes, std::uint8_t seed,
                                        Stream const& stream) {
  return fill(dst, bytes, seed, true, stream, "fill_pattern");
}

// ---- copies and uploads ------------------------------------------------------------
static expected<void, Error> copy(void* dst, void const* src, std::uint64_t bytes,
                                       hipMemcpyKind kind, Stream const& stream, char const* op) {
  if (!bytes) return {};
  if (!dst || !src) return unexpected(make_error(ErrorCode::InvalidArgument, op, "null pointer"));
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  return check(hipMemcpyAsync(dst, src, bytes, kind, stream.native()), op);
}

expected<void, Error> copy_h2d(void* dst, void const* src, std::uint64_t bytes,
                                    Stream const& stream) {
  return copy(dst, src, bytes, hipMemcpyHostToDevice, stream, "copy_h2d");
}
expected<void, Error> copy_d2h(void* dst, void const* src, std::uint64_t bytes,
                                    Stream const& stream) {
  return copy(dst, src, bytes, hipMemcpyDeviceToHost, stream, "copy_d2h");
}
expected<void, Error> copy_d2d(void* dst, void const* src, std::uint64_t bytes,
                                    Stream const& stream) {
  return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream, "copy_d2d");
}
expected<void, Error> copy_h2d(void* dst, std::span<std::byte const> src, Stream const& stream) {
  return copy_h2d(dst, src.data(), src.size(), stream);
}
expected<void, Error> copy_d2h(std::span<std::byte> dst, void const* src, Stream const& stream) {
  return copy_d2h(dst.data(), src, dst.size(), stream);
}

expected<DeviceBuffer, Error> upload(std::span<std::byte const> host, Stream const& stream) {
  if (host.empty())
    return unexpected(make_error(ErrorCode::InvalidArgument, "upload", "empty payload"));
  auto buffer = DeviceBuffer::allocate(host.size(), stream.device());
  if (!buffer) return unexpected(buffer.error());
  if (auto st = copy_h2d(buffer->data(), host, stream); !st) return unexpected(st.error());
  return buffer;
}

PrefillWeight TiledWeight::weight() const {
  PrefillWeight w;
  w.codes = codes.data();
  w.scales = scales.data();
  w.layout = layout;
  w.quantizer = quantizer;
  w.n = n;
  w.k = k;
  w.padded_n = (n + 7) / 8 * 8;
  w.padded_k = (k + 255) / 256 * 256;
  w.codes_bytes = codes.bytes();
  w.scales_bytes = scales.bytes();
  return w;
}

static expected<TiledWeight, Error> upload_blocks(std::span<std::byte const> blocks,
                                                       std::uint32_t n, std::uint32_t k,
                                                       std::uint16_t layout, bool q6,
                                                       Stream const& stream) {
  const char* op = q6 ? "upload.q6k_blocks" : "upload.q4k_blocks";
  const std::uint64_t per = q6 ? 210 : 144;
  if (!n || !k || k % 256 || blocks.size() != std::uint64_t(n) * (k / 256) * per)
    return unexpected(make_error(ErrorCode::InvalidArgument, op, "block count mismatch"));
  const std::uint32_t pn = (n + 7) / 8 * 8;
  const std::uint64_t cb = qw38_code_bytes(layout, pn, k), sb = qw38_scale_bytes(layout, pn, k);
  if (!cb || !sb) return unexpected(make_error(ErrorCode::InvalidArgument, op, "unknown layout"));
  auto staged = upload(blocks, stream);
  if (!staged) return unexpected(staged.error());
  auto codes = DeviceBuffer::allocate(cb, stream.device());
  if (!codes) return unexpected(codes.error());
  auto scales = DeviceBuffer::allocate(sb, stream.device());
  if (!scales) return unexpected(scales.error());
  auto guard = stream.activate();
  if (!guard) return unexpected(guard.error());
  const int st = q6 ? qw38_repack_q6k_blocks(staged->data(), staged->bytes(), n, k, codes->data(),
                                             cb, scales->data(), sb, stream.native())
                    : qw38_repack_q4k_blocks(staged->data(), staged->bytes(), n, k, layout,
                                             codes->data(), cb, scales->data(), sb, stream.native());
  if (auto r = from_abi(st); !r) return unexpected(r.error());
  // the staging buffer is released only after the repack has consumed it
  if (auto r = stream.sync(); !r) return unexpected(r.error());
  TiledWeight t;
  t.codes = std::move(*codes);
  t.scales = std::move(*scales);
  t.layout = layout;
  t.quantizer = q6 ? QW38_QUANTIZER_Q6K : QW38_QUANTIZER_Q4K;
  t.n = n;
  t.k = k;
  return t;
}

expected<TiledWeight, Error> upload_q4k_blocks(std::span<std::byte const> blocks,
                                                    std::uint32_t n, std::uint32_t k,
                                                    std::uint16_t layout, Stream const& stream) {
  return upload_blocks(blocks, n, k, layout, false, stream);
}

expected<TiledWeight, Error> upload_q6k_blocks(std::span<std::byte const> blocks,
                                                    std::uint32_t n, std::uint32_t k,
                                                    Stream const& stream) {
  return upload_blocks(blocks, n, k, QW38_LAYOUT_Q6K_WAVE64, true, stream);
}

}  // namespace qw38::cuda
