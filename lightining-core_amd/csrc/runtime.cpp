// runtime.cpp -- device layer, capability contracts, trace ring and the
// reference's runtime C ABI (include/lightning_core/lightning_core.h:113-137)
// backed by HIP.
//
// Reference behaviour kept (src/runtime.cpp):
//   * trace ring of 4096 events, off by default (:63-99, :620-653);
//   * dispatch detail encoding requested | selected << 4 | fallback << 8
//     (:703-748), decoding rejects unknown device values;
//   * capability / interface-contract derivation (:492-618);
//   * sync policy modes auto / always / never (:425-490).
// HIP replaces CUDA/Metal: malloc/free/memcpy map to hipMalloc/hipFree/
// hipMemcpy, deviceSynchronize drains the backend stream, the memory model is
// native-device, and the preferred device is hip when a gfx950 is visible.
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "kernels.hpp"
#include "lc_internal.hpp"
#include "tune.hpp"

namespace lchip {

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
namespace {
thread_local std::string t_last_error;
}

void setLastError(const std::string& msg) { t_last_error = msg; }
const char* lastError() { return t_last_error.c_str(); }

Status fail(Status st, const std::string& msg) {
  t_last_error = msg;
  return st;
}

Status failHip(hipError_t e, const char* what) {
  // The error is reported here; clear HIP's per-thread last error so the next
  // launch's hipGetLastError() does not report it again (a failed hipMalloc
  // would otherwise fail the next kernel launch).
  (void)hipGetLastError();
  Status st = Status::kDriverError;
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
    st = Status::kOutOfMemory;
  } else if (e == hipErrorInvalidValue) {
    st = Status::kInvalidValue;
  } else if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) {
    st = Status::kNotSupported;
  }
  t_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return st;
}

// ---------------------------------------------------------------------------
// trace ring
// ---------------------------------------------------------------------------
namespace {
std::atomic<bool> g_trace_enabled{false};
std::mutex g_trace_mu;
std::vector<lcRuntimeTraceEvent> g_trace;
std::size_t g_trace_write = 0;
std::atomic<int> g_sync_mode{LC_SYNC_AUTO};
std::atomic<bool> g_sync_trace_boundary{false};

uint64_t nowNs() {
  return static_cast<uint64_t>(
      std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
          .count());
}
}  // namespace

void traceRecord(TraceEventType type, Status st, std::size_t size_bytes, int d0, int d1) {
  if (!g_trace_enabled.load(std::memory_order_relaxed)) {
    return;
  }
  lcRuntimeTraceEvent ev{};
  ev.type = static_cast<int>(type);
  ev.status = toLc(st);
  ev.timestamp_ns = nowNs();
  ev.size_bytes = size_bytes;
  ev.detail0 = d0;
  ev.detail1 = d1;
  std::lock_guard<std::mutex> lock(g_trace_mu);
  if (g_trace.size() < kTraceCapacity) {
    g_trace.push_back(ev);
    return;
  }
  g_trace[g_trace_write] = ev;
  g_trace_write = (g_trace_write + 1) % kTraceCapacity;
}

int encodeDispatch(Device requested, Device selected, bool fallback) {
  return (static_cast<int>(requested) & 0x0F) | ((static_cast<int>(selected) & 0x0F) << 4) | (fallback ? (1 << 8) : 0);
}

void traceOpDispatch(TraceOp op, Device requested, Device selected, bool fallback, std::size_t workload_hint) {
  traceRecord(TraceEventType::kOpDispatch, Status::kSuccess, workload_hint, static_cast<int>(op),
              encodeDispatch(requested, selected, fallback));
}

// ---------------------------------------------------------------------------
// HIP context
// ---------------------------------------------------------------------------
namespace {
std::once_flag g_ctx_once;
HipContext* g_ctx = nullptr;  // intentionally never destroyed (process lifetime)
Status g_ctx_status = Status::kNotInitialized;
std::string g_ctx_error;

void initContext() {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) {
    g_ctx_status = Status::kNotSupported;
    g_ctx_error = "hip device not available (no visible HIP device)";
    return;
  }
  // Use the first visible gfx950; kernels are built for gfx950 only.
  for (int d = 0; d < count; ++d) {
    hipDeviceProp_t props{};
    if (hipGetDeviceProperties(&props, d) != hipSuccess) {
      continue;
    }
    if (std::strncmp(props.gcnArchName, "gfx950", 6) != 0) {
      continue;
    }
    auto* ctx = new HipContext();
    ctx->device = d;
    ctx->props = props;
    if (hipSetDevice(d) != hipSuccess || hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
      delete ctx;
      g_ctx_status = Status::kDriverError;
      g_ctx_error = "failed to create the backend HIP stream";
      return;
    }
    g_ctx = ctx;
    g_ctx_status = Status::kSuccess;
    return;
  }
  g_ctx_status = Status::kNotSupported;
  g_ctx_error = "hip device not available (no gfx950 device visible; kernels are built for gfx950 only)";
}
}  // namespace

HipContext* hipContext(Status* st) {
  ensureRuntimeProfileLoaded();
  std::call_once(g_ctx_once, initContext);
  if (g_ctx == nullptr) {
    if (st != nullptr) {
      *st = fail(g_ctx_status, g_ctx_error);
    }
    return nullptr;
  }
  // Host threads other than the first may have another current device.
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != g_ctx->device) {
    (void)hipSetDevice(g_ctx->device);
  }
  if (st != nullptr) {
    *st = Status::kSuccess;
  }
  return g_ctx;
}

bool hipAvailable() { return hipContext(nullptr) != nullptr; }

Status DeviceBuffer::ensure(std::size_t bytes, bool zero) {
  if (bytes <= bytes_ && ptr_ != nullptr) {
    return Status::kSuccess;
  }
  const std::size_t old = bytes_;
  reset();
  std::size_t want = bytes;
  if (old != 0) {
    want = std::max(bytes, old + old / 2);
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    // retry with the exact size before giving up
    e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
      return failHip(e, "hipMalloc");
    }
    want = bytes;
  }
  ptr_ = p;
  bytes_ = want;
  if (zero) {
    // the null stream does not order with the non-blocking backend stream:
    // finish the fill before any kernel can read the buffer
    e = hipMemset(ptr_, 0, bytes_);
    if (e == hipSuccess) {
      e = hipDeviceSynchronize();
    }
    if (e != hipSuccess) {
      return failHip(e, "hipMemset");
    }
  }
  return Status::kSuccess;
}

void DeviceBuffer::reset() {
  if (ptr_ != nullptr) {
    (void)hipFree(ptr_);
  }
  ptr_ = nullptr;
  bytes_ = 0;
}

Status PinnedBuffer::ensure(std::size_t bytes) {
  if (bytes <= bytes_ && ptr_ != nullptr) {
    return Status::kSuccess;
  }
  const std::size_t want = std::max(bytes, bytes_ + bytes_ / 2);
  reset();
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
  if (e != hipSuccess) {
    return failHip(e, "hipHostMalloc");
  }
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, p, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(p);
    return failHip(e, "hipHostGetDevicePointer");
  }
  ptr_ = p;
  dev_ = d;
  bytes_ = want;
  return Status::kSuccess;
}

void PinnedBuffer::reset() {
  if (ptr_ != nullptr) {
    (void)hipHostFree(ptr_);  // synchronises the device: no copy can still use it
  }
  ptr_ = nullptr;
  dev_ = nullptr;
  bytes_ = 0;
}

Status upload(HipContext* ctx, void* dst, const void* src, std::size_t bytes) {
  LC_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  return Status::kSuccess;
}

Status download(HipContext* ctx, void* dst, const void* src, std::size_t bytes) {
  LC_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  return Status::kSuccess;
}

namespace {
// Bookkeeping after the stream has drained: in-flight counts restart, and a
// failure a kernel recorded since the last sync becomes an error.
Status afterSync(HipContext* ctx) {
  ctx->matmul_inflight = 0;
  ctx->attention_inflight = 0;
  if (int* word = static_cast<int*>(ctx->gemm_fail.get())) {
    if (__atomic_exchange_n(word, 0, __ATOMIC_ACQ_REL) != 0) {
      // The stream is idle, so the launch whose wait ran out has completed:
      // zero the flags a late publisher may have set with that launch's
      // epoch, so a replay of a captured launch (which reuses its epoch)
      // cannot take them for ready.
      if (void* flags = ctx->gemm_flags.get()) {
        LC_HIP_TRY(hipMemsetAsync(flags, 0, ctx->gemm_flags.size(), ctx->stream));
        LC_HIP_TRY(hipStreamSynchronize(ctx->stream));
      }
      return fail(Status::kDriverError,
                  "matmul: a stream-K workgroup's bounded wait for a partial tile ran out "
                  "(CJ_HIP_STREAMK_SPIN_LIMIT); the result of that launch is invalid");
    }
  }
  return Status::kSuccess;
}
}  // namespace

Status syncStream(HipContext* ctx) {
  LC_HIP_TRY(hipStreamSynchronize(ctx->stream));
  return afterSync(ctx);
}

Status prepareDoneFlag(HipContext* ctx, unsigned** flag_dev, unsigned** count_dev, unsigned* seq) {
  if (ctx->done_flag.get() == nullptr) {
    LC_TRY(ctx->done_flag.ensure(64));
    __atomic_store_n(static_cast<unsigned*>(ctx->done_flag.get()), 0u, __ATOMIC_RELEASE);
    LC_TRY(ctx->done_count.ensure(64, true));
    LC_HIP_TRY(hipStreamSynchronize(ctx->stream));  // the zeroed counter is in place
  }
  ctx->done_seq = ctx->done_seq + 1 == 0 ? 1 : ctx->done_seq + 1;  // never 0, the initial word
  *flag_dev = static_cast<unsigned*>(ctx->done_flag.device());
  *count_dev = ctx->done_count.as<unsigned>();
  *seq = ctx->done_seq;
  return Status::kSuccess;
}

Status waitDoneFlag(HipContext* ctx, unsigned seq) {
  // Spin budget: 200 ms, or CJ_HIP_DONE_WAIT_US (read once; 0 takes the
  // stream-sync path below at once).
  static const long long budget_us = [] {
    const char* v = std::getenv("CJ_HIP_DONE_WAIT_US");
    return v != nullptr ? std::atoll(v) : 200000LL;
  }();
  const unsigned* word = static_cast<const unsigned*>(ctx->done_flag.get());
  const auto t0 = std::chrono::steady_clock::now();
  for (;;) {
    if (__atomic_load_n(word, __ATOMIC_ACQUIRE) == seq) {
      return afterSync(ctx);
    }
    if (std::chrono::steady_clock::now() - t0 >= std::chrono::microseconds(budget_us)) {
      break;
    }
  }
  // Not seen in time: the stream sync reports a failed launch; after one
  // that completed, its results are in place whether or not the word came
  // (a counter left off zero by an earlier failed launch keeps it away), so
  // the counter is re-zeroed for the next call.
  LC_TRY(syncStream(ctx));
  if (__atomic_load_n(word, __ATOMIC_ACQUIRE) != seq) {
    LC_HIP_TRY(hipMemsetAsync(ctx->done_count.get(), 0, ctx->done_count.size(), ctx->stream));
    LC_HIP_TRY(hipStreamSynchronize(ctx->stream));
  }
  return Status::kSuccess;
}

// Synchronous downloads of small results: one kernel copies the device buffers into the pinned staging and
// raises the completion flag; the host waits on the flag and copies out.  A
// pageable download and a stream sync cost ~10 us each at these sizes.
Status stagedDownload(HipContext* ctx, const StagedOut* outs, int count) {
  std::size_t at[4] = {0, 0, 0, 0};
  std::size_t total = 0;
  for (int c = 0; c < count; ++c) {
    at[c] = total;
    total += roundUp(outs[c].n, 64);
  }
  LC_TRY(ctx->pinned.ensure(total * sizeof(float)));
  unsigned* flag_dev = nullptr;
  unsigned* count_dev = nullptr;
  unsigned seq = 0;
  LC_TRY(prepareDoneFlag(ctx, &flag_dev, &count_dev, &seq));
  float* dev = static_cast<float*>(ctx->pinned.device());
  kern::CopySegsF32 segs{};
  for (int c = 0; c < count; ++c) {
    segs.seg[c] = kern::CopySegF32{outs[c].src, dev + at[c], outs[c].n};
  }
  segs.count = count;
  const hipError_t e = kern::copySegsF32(segs, ctx->stream, count_dev, flag_dev, seq);
  if (e != hipSuccess) {
    return failHip(e, "staged download copy");
  }
  LC_TRY(waitDoneFlag(ctx, seq));
  const float* stage = static_cast<const float*>(ctx->pinned.get());
  for (int c = 0; c < count; ++c) {
    std::memcpy(outs[c].dst, stage + at[c], outs[c].n * sizeof(float));
  }
  return Status::kSuccess;
}

Status noteEnqueued(HipContext* ctx, TraceOp op, std::size_t launches) {
  const bool mm = op == TraceOp::kMatMul;
  std::size_t& count = mm ? ctx->matmul_inflight : ctx->attention_inflight;
  count += launches;
  if (count < (mm ? kMatMulMaxInflight : kAttentionMaxInflight)) {
    return Status::kSuccess;
  }
  const std::size_t was = count;
  const Status st = syncStream(ctx);
  traceRecord(TraceEventType::kDeviceSynchronize, st, was, static_cast<int>(op), 1);
  return st;
}

Status nextStreamKEpoch(HipContext* ctx, int* epoch) {
  if (ctx->gemm_epoch >= (1 << 30)) {
    // wrap: no flag may still hold an epoch the new sequence reuses
    LC_HIP_TRY(hipMemsetAsync(ctx->gemm_flags.get(), 0, ctx->gemm_flags.size(), ctx->stream));
    ctx->gemm_epoch = 0;
  }
  *epoch = ++ctx->gemm_epoch;
  return Status::kSuccess;
}

int streamKSpinLimit() {
  if (const char* env = std::getenv("CJ_HIP_STREAMK_SPIN_LIMIT")) {
    char* end = nullptr;
    const long v = std::strtol(env, &end, 10);
    if (end != env && *end == '\0' && v >= 0 && v <= (1L << 30)) {
      return static_cast<int>(v);
    }
  }
  return kern::kStreamKSpinLimit;
}

// ---------------------------------------------------------------------------
// runtime surface (src/runtime.cpp:193-618 semantics)
// ---------------------------------------------------------------------------
namespace {

Status mallocDevice(void** ptr, std::size_t size_bytes) {
  if (ptr == nullptr || size_bytes == 0) {
    traceRecord(TraceEventType::kMallocDevice, Status::kInvalidValue, size_bytes);
    return Status::kInvalidValue;
  }
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx == nullptr) {
    *ptr = nullptr;
  } else {
    hipError_t e = hipMalloc(ptr, size_bytes);
    st = (e == hipSuccess) ? Status::kSuccess : failHip(e, "hipMalloc");
  }
  traceRecord(TraceEventType::kMallocDevice, st, size_bytes);
  return st;
}

Status freeDevice(void* ptr) {
  Status st = Status::kSuccess;
  if (ptr != nullptr) {
    HipContext* ctx = hipContext(&st);
    if (ctx != nullptr) {
      hipError_t e = hipFree(ptr);
      st = (e == hipSuccess) ? Status::kSuccess : failHip(e, "hipFree");
    }
  }
  traceRecord(TraceEventType::kFreeDevice, st);
  return st;
}

Status memcpyKind(void* dst, const void* src, std::size_t size_bytes, lcMemcpyKind kind) {
  if (dst == nullptr || src == nullptr) {
    traceRecord(TraceEventType::kMemcpy, Status::kInvalidValue, size_bytes, static_cast<int>(kind));
    return Status::kInvalidValue;
  }
  Status st = Status::kSuccess;
  if (kind == LC_MEMCPY_HOST_TO_HOST) {
    std::memcpy(dst, src, size_bytes);
  } else {
    HipContext* ctx = hipContext(&st);
    if (ctx != nullptr) {
      hipMemcpyKind hk = hipMemcpyDefault;
      switch (kind) {
        case LC_MEMCPY_HOST_TO_DEVICE:
          hk = hipMemcpyHostToDevice;
          break;
        case LC_MEMCPY_DEVICE_TO_HOST:
          hk = hipMemcpyDeviceToHost;
          break;
        case LC_MEMCPY_DEVICE_TO_DEVICE:
          hk = hipMemcpyDeviceToDevice;
          break;
        default:
          break;
      }
      // Ordered after all work queued on the backend stream.
      hipError_t e = hipMemcpyAsync(dst, src, size_bytes, hk, ctx->stream);
      if (e == hipSuccess) {
        e = hipStreamSynchronize(ctx->stream);
      }
      st = (e == hipSuccess) ? Status::kSuccess : failHip(e, "hipMemcpy");
    }
  }
  traceRecord(TraceEventType::kMemcpy, st, size_bytes, static_cast<int>(kind));
  return st;
}

Status deviceSynchronize() {
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx != nullptr) {
    st = syncStream(ctx);
  }
  traceRecord(TraceEventType::kDeviceSynchronize, st);
  return st;
}

Device preferredDevice(int workload) {
  const Device selected = hipAvailable() ? Device::kHIP : Device::kCPU;
  traceRecord(TraceEventType::kPreferredDeviceFor, Status::kSuccess, 0, workload, static_cast<int>(selected));
  return selected;
}

lcBackendCapabilities capabilities(lcDeviceKind device) {
  lcBackendCapabilities caps{};
  caps.device = device;
  caps.runtime_trace_surface = 1;
  caps.sync_policy_surface = 1;
  caps.profiling_surface = 0;
  switch (device) {
    case LC_DEVICE_CPU:
      // The host is always there, but this library runs no compute on it: the
      // reference's own CPU backend serves device "cpu".
      caps.built = 1;
      caps.available = 1;
      caps.compute_surface = 0;
      caps.memory_surface = 0;
      caps.sync_surface = 0;
      caps.memory_model = LC_MEMORY_HOST_MANAGED_COMPAT;
      break;
    case LC_DEVICE_CUDA:
      caps.built = 0;
      caps.available = 0;
      caps.memory_model = LC_MEMORY_NATIVE_DEVICE;
      traceRecord(TraceEventType::kIsCudaAvailable, Status::kSuccess, 0, 0);
      break;
    case LC_DEVICE_METAL:
      caps.built = 0;
      caps.available = 0;
      caps.memory_model = LC_MEMORY_HOST_MANAGED_COMPAT;
      traceRecord(TraceEventType::kIsMetalAvailable, Status::kSuccess, 0, 0);
      break;
    case LC_DEVICE_HIP:
    default:
      caps.built = 1;
      caps.available = hipAvailable() ? 1 : 0;
      caps.compute_surface = 1;
      caps.memory_surface = 1;
      caps.sync_surface = 1;
      caps.profiling_surface = 1;  // hipEvent timers on the backend stream
      caps.memory_model = LC_MEMORY_NATIVE_DEVICE;
      break;
  }
  return caps;
}

const char* computeTag(lcDeviceKind d) {
  switch (d) {
    case LC_DEVICE_HIP:
      return "hip.compute.dispatch";
    case LC_DEVICE_CUDA:
      return "cuda.runtime.dispatch";
    case LC_DEVICE_METAL:
      return "metal.compute.dispatch";
    default:
      return "cpu.eager.dispatch";
  }
}
const char* memoryTag(lcDeviceKind d) {
  switch (d) {
    case LC_DEVICE_HIP:
      return "hip.device_memory";
    case LC_DEVICE_CUDA:
      return "cuda.memory";
    case LC_DEVICE_METAL:
      return "metal.host_managed_memory";
    default:
      return "cpu.host_memory";
  }
}
const char* syncTag(lcDeviceKind d) {
  switch (d) {
    case LC_DEVICE_HIP:
      return "hip.stream_event_sync";
    case LC_DEVICE_CUDA:
      return "cuda.device_sync";
    case LC_DEVICE_METAL:
      return "metal.command_sync";
    default:
      return "cpu.noop_sync";
  }
}

lcBackendInterfaceContract contract(lcDeviceKind device) {
  const lcBackendCapabilities caps = capabilities(device);
  lcBackendInterfaceContract c{};
  c.device = device;
  c.capabilities = caps;
  c.compute.available = caps.compute_surface;
  c.compute.op_dispatch_trace_surface = caps.runtime_trace_surface;
  c.compute.driver_tag = computeTag(device);
  c.memory.available = (device == LC_DEVICE_CPU) ? 1 : caps.memory_surface;
  c.memory.allocator_surface = caps.memory_surface;
  c.memory.memcpy_surface = 1;
  c.memory.memory_model = caps.memory_model;
  c.memory.driver_tag = memoryTag(device);
  c.sync.available = (device == LC_DEVICE_CPU) ? 1 : caps.sync_surface;
  c.sync.sync_policy_surface = caps.sync_policy_surface;
  c.sync.trace_sync_boundary_surface = caps.sync_policy_surface;
  c.sync.driver_tag = syncTag(device);
  c.profiler.available = caps.runtime_trace_surface;
  c.profiler.runtime_trace_surface = caps.runtime_trace_surface;
  c.profiler.op_dispatch_trace_surface = caps.runtime_trace_surface;
  c.profiler.trace_capacity = kTraceCapacity;
  c.profiler.driver_tag = "runtime.trace.ring";
  return c;
}

}  // namespace
}  // namespace lchip

using namespace lchip;

extern "C" {

lcError_t lcMalloc(void** ptr, size_t size_bytes) { return toLc(mallocDevice(ptr, size_bytes)); }
lcError_t lcFree(void* ptr) { return toLc(freeDevice(ptr)); }
lcError_t lcMemcpy(void* dst, const void* src, size_t size_bytes, lcMemcpyKind kind) {
  return toLc(memcpyKind(dst, src, size_bytes, kind));
}
lcError_t lcDeviceSynchronize(void) { return toLc(deviceSynchronize()); }

lcError_t lcGetDeviceCount(int* count) {
  if (count == nullptr) {
    traceRecord(TraceEventType::kGetDeviceCount, Status::kInvalidValue);
    return LC_INVALID_VALUE;
  }
  const bool ok = hipAvailable();
  *count = ok ? 1 : 0;
  const Status st = ok ? Status::kSuccess : Status::kNotSupported;
  traceRecord(TraceEventType::kGetDeviceCount, st, 0, *count);
  return toLc(st);
}

lcError_t lcGetPreferredDeviceForInference(lcDeviceKind* device) {
  if (device == nullptr) {
    return LC_INVALID_VALUE;
  }
  *device = static_cast<lcDeviceKind>(static_cast<int>(preferredDevice(1)));
  return LC_SUCCESS;
}

lcError_t lcGetPreferredDeviceForTraining(lcDeviceKind* device) {
  if (device == nullptr) {
    return LC_INVALID_VALUE;
  }
  *device = static_cast<lcDeviceKind>(static_cast<int>(preferredDevice(0)));
  return LC_SUCCESS;
}

int lcIsCudaAvailable(void) {
  traceRecord(TraceEventType::kIsCudaAvailable, Status::kSuccess, 0, 0);
  return 0;
}

int lcIsMetalAvailable(void) {
  traceRecord(TraceEventType::kIsMetalAvailable, Status::kSuccess, 0, 0);
  return 0;
}

int lcIsHipAvailable(void) { return hipAvailable() ? 1 : 0; }

lcMemoryModel lcGetMemoryModel(void) { return LC_MEMORY_NATIVE_DEVICE; }

const char* lcGetMemoryModelName(lcMemoryModel model) {
  return model == LC_MEMORY_NATIVE_DEVICE ? "native-device" : "host-managed-compat";
}

lcError_t lcSetDefaultSyncPolicy(lcSyncPolicy policy) {
  g_sync_mode.store(static_cast<int>(policy.mode), std::memory_order_relaxed);
  g_sync_trace_boundary.store(policy.trace_sync_boundary != 0, std::memory_order_relaxed);
  return LC_SUCCESS;
}

lcSyncPolicy lcGetDefaultSyncPolicy(void) {
  lcSyncPolicy p{};
  const int raw = g_sync_mode.load(std::memory_order_relaxed);
  p.mode = (raw == LC_SYNC_ALWAYS || raw == LC_SYNC_NEVER) ? static_cast<lcSyncMode>(raw) : LC_SYNC_AUTO;
  p.trace_sync_boundary = g_sync_trace_boundary.load(std::memory_order_relaxed) ? 1 : 0;
  return p;
}

lcError_t lcApplySyncPolicy(lcSyncPolicy policy) {
  Status st = Status::kSuccess;
  switch (policy.mode) {
    case LC_SYNC_NEVER:
      break;
    case LC_SYNC_ALWAYS:
      st = deviceSynchronize();
      break;
    case LC_SYNC_AUTO:
    default:
      if (hipAvailable()) {
        st = deviceSynchronize();
      }
      break;
  }
  traceRecord(TraceEventType::kApplySyncPolicy, st, 0, static_cast<int>(policy.mode),
              policy.trace_sync_boundary ? 1 : 0);
  return toLc(st);
}

lcError_t lcApplyDefaultSyncPolicy(void) { return lcApplySyncPolicy(lcGetDefaultSyncPolicy()); }

lcError_t lcGetBackendCapabilities(lcDeviceKind device, lcBackendCapabilities* out_caps) {
  if (out_caps == nullptr || !validDevice(device)) {
    return LC_INVALID_VALUE;
  }
  *out_caps = capabilities(device);
  return LC_SUCCESS;
}

lcError_t lcGetActiveBackendCapabilities(lcBackendCapabilities* out_caps) {
  if (out_caps == nullptr) {
    return LC_INVALID_VALUE;
  }
  *out_caps = capabilities(static_cast<lcDeviceKind>(static_cast<int>(preferredDevice(1))));
  return LC_SUCCESS;
}

lcError_t lcGetBackendInterfaceContract(lcDeviceKind device, lcBackendInterfaceContract* out_contract) {
  if (out_contract == nullptr || !validDevice(device)) {
    return LC_INVALID_VALUE;
  }
  *out_contract = contract(device);
  return LC_SUCCESS;
}

lcError_t lcGetActiveBackendInterfaceContract(lcBackendInterfaceContract* out_contract) {
  if (out_contract == nullptr) {
    return LC_INVALID_VALUE;
  }
  *out_contract = contract(static_cast<lcDeviceKind>(static_cast<int>(preferredDevice(1))));
  return LC_SUCCESS;
}

lcError_t lcGetApiVersion(int* out_major, int* out_minor, int* out_patch) {
  if (out_major == nullptr || out_minor == nullptr || out_patch == nullptr) {
    return LC_INVALID_VALUE;
  }
  *out_major = LC_API_VERSION_MAJOR;
  *out_minor = LC_API_VERSION_MINOR;
  *out_patch = LC_API_VERSION_PATCH;
  return LC_SUCCESS;
}

const char* lcGetApiVersionString(void) { return LC_API_VERSION_STRING; }

size_t lcGetStructSize(lcStructId struct_id) {
  switch (struct_id) {
    case LC_STRUCT_BACKEND_CAPABILITIES:
      return sizeof(lcBackendCapabilities);
    case LC_STRUCT_COMPUTE_INTERFACE_CONTRACT:
      return sizeof(lcComputeInterfaceContract);
    case LC_STRUCT_MEMORY_INTERFACE_CONTRACT:
      return sizeof(lcMemoryInterfaceContract);
    case LC_STRUCT_SYNC_INTERFACE_CONTRACT:
      return sizeof(lcSyncInterfaceContract);
    case LC_STRUCT_PROFILER_INTERFACE_CONTRACT:
      return sizeof(lcProfilerInterfaceContract);
    case LC_STRUCT_BACKEND_INTERFACE_CONTRACT:
      return sizeof(lcBackendInterfaceContract);
    default:
      return 0;
  }
}

int lcCheckStructSize(lcStructId struct_id, size_t observed_size) {
  const size_t expected = lcGetStructSize(struct_id);
  return (expected != 0 && observed_size == expected) ? 1 : 0;
}

const char* lcBackendName(void) {
  traceRecord(TraceEventType::kBackendName, Status::kSuccess);
  return hipAvailable() ? "hip" : "cpu";
}

const char* lcGetErrorString(lcError_t error) {
  switch (error) {
    case LC_SUCCESS:
      return "success";
    case LC_NOT_INITIALIZED:
      return "not initialized";
    case LC_INVALID_VALUE:
      return "invalid value";
    case LC_OUT_OF_MEMORY:
      return "out of memory";
    case LC_NOT_SUPPORTED:
      return "not supported";
    case LC_DRIVER_ERROR:
      return "driver error";
    case LC_UNKNOWN:
    default:
      return "unknown error";
  }
}

const char* lcGetLastErrorMessage(void) { return lastError(); }

void lcSetRuntimeTraceEnabled(int enabled) { g_trace_enabled.store(enabled != 0, std::memory_order_relaxed); }
int lcIsRuntimeTraceEnabled(void) { return g_trace_enabled.load(std::memory_order_relaxed) ? 1 : 0; }

void lcClearRuntimeTraceEvents(void) {
  std::lock_guard<std::mutex> lock(g_trace_mu);
  g_trace.clear();
  g_trace_write = 0;
}

size_t lcGetRuntimeTraceEvents(lcRuntimeTraceEvent* out, size_t capacity) {
  std::lock_guard<std::mutex> lock(g_trace_mu);
  const size_t n = g_trace.size();
  if (out == nullptr) {
    return n;
  }
  // chronological order: oldest first (the write index is the oldest slot once wrapped)
  const size_t start = (n < kTraceCapacity) ? 0 : g_trace_write;
  size_t written = 0;
  for (size_t i = 0; i < n && written < capacity; ++i) {
    out[written++] = g_trace[(start + i) % n];
  }
  return written;
}

size_t lcGetRuntimeTraceEventCapacity(void) { return kTraceCapacity; }

const char* lcRuntimeTraceEventTypeName(int type) {
  switch (static_cast<TraceEventType>(type)) {
    case TraceEventType::kMallocDevice:
      return "malloc_device";
    case TraceEventType::kFreeDevice:
      return "free_device";
    case TraceEventType::kMemcpy:
      return "memcpy";
    case TraceEventType::kDeviceSynchronize:
      return "device_synchronize";
    case TraceEventType::kApplySyncPolicy:
      return "apply_sync_policy";
    case TraceEventType::kGetDeviceCount:
      return "get_device_count";
    case TraceEventType::kIsCudaAvailable:
      return "is_cuda_available";
    case TraceEventType::kIsMetalAvailable:
      return "is_metal_available";
    case TraceEventType::kPreferredDeviceFor:
      return "preferred_device_for";
    case TraceEventType::kOpDispatch:
      return "op_dispatch";
    case TraceEventType::kBackendName:
    default:
      return "backend_name";
  }
}

const char* lcRuntimeTraceOpKindName(int op) {
  switch (static_cast<TraceOp>(op)) {
    case TraceOp::kMatMul:
      return "matmul";
    case TraceOp::kVectorAdd:
      return "vector_add";
    case TraceOp::kMatrixSub:
      return "matrix_sub";
    case TraceOp::kMatrixDiv:
      return "matrix_div";
    case TraceOp::kConv2dNchw:
      return "conv2d_nchw";
    case TraceOp::kAttentionForward:
      return "attention_forward";
    case TraceOp::kUnknown:
    default:
      return "unknown";
  }
}

int lcEncodeRuntimeTraceDispatchDetail(lcDeviceKind requested, lcDeviceKind selected, int fallback) {
  return encodeDispatch(fromLc(requested), fromLc(selected), fallback != 0);
}

int lcDecodeRuntimeTraceDispatchDetail(int encoded, lcDeviceKind* requested, lcDeviceKind* selected, int* fallback) {
  if (requested == nullptr || selected == nullptr || fallback == nullptr) {
    return 0;
  }
  const int r = encoded & 0x0F;
  const int s = (encoded >> 4) & 0x0F;
  if (r > LC_DEVICE_HIP || s > LC_DEVICE_HIP) {
    return 0;
  }
  *requested = static_cast<lcDeviceKind>(r);
  *selected = static_cast<lcDeviceKind>(s);
  *fallback = ((encoded >> 8) & 1) != 0 ? 1 : 0;
  return 1;
}

lcError_t lcHipGetDeviceInfo(lcHipDeviceInfo* out) {
  if (out == nullptr) {
    return LC_INVALID_VALUE;
  }
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx == nullptr) {
    return toLc(st);
  }
  std::memset(out, 0, sizeof(*out));
  std::strncpy(out->name, ctx->props.name, sizeof(out->name) - 1);
  std::strncpy(out->gcn_arch, ctx->props.gcnArchName, sizeof(out->gcn_arch) - 1);
  out->compute_units = ctx->props.multiProcessorCount;
  out->max_clock_khz = ctx->props.clockRate;
  out->total_memory_bytes = ctx->props.totalGlobalMem;
  out->l2_cache_bytes = static_cast<size_t>(ctx->props.l2CacheSize);
  return LC_SUCCESS;
}

struct lcHipTimer {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

lcError_t lcHipTimerCreate(lcHipTimer** out) {
  if (out == nullptr) {
    return LC_INVALID_VALUE;
  }
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx == nullptr) {
    return toLc(st);
  }
  auto* t = new lcHipTimer();
  if (hipEventCreate(&t->start) != hipSuccess || hipEventCreate(&t->stop) != hipSuccess) {
    delete t;
    return toLc(fail(Status::kDriverError, "hipEventCreate failed"));
  }
  *out = t;
  return LC_SUCCESS;
}

lcError_t lcHipTimerDestroy(lcHipTimer* t) {
  if (t == nullptr) {
    return LC_INVALID_VALUE;
  }
  (void)hipEventDestroy(t->start);
  (void)hipEventDestroy(t->stop);
  delete t;
  return LC_SUCCESS;
}

lcError_t lcHipTimerStart(lcHipTimer* t) {
  if (t == nullptr) {
    return LC_INVALID_VALUE;
  }
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx == nullptr) {
    return toLc(st);
  }
  hipError_t e = hipEventRecord(t->start, ctx->stream);
  return e == hipSuccess ? LC_SUCCESS : toLc(failHip(e, "hipEventRecord"));
}

lcError_t lcHipTimerStop(lcHipTimer* t, float* elapsed_ms) {
  if (t == nullptr || elapsed_ms == nullptr) {
    return LC_INVALID_VALUE;
  }
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx == nullptr) {
    return toLc(st);
  }
  hipError_t e = hipEventRecord(t->stop, ctx->stream);
  if (e == hipSuccess) {
    e = hipEventSynchronize(t->stop);
  }
  if (e == hipSuccess) {
    e = hipEventElapsedTime(elapsed_ms, t->start, t->stop);
  }
  return e == hipSuccess ? LC_SUCCESS : toLc(failHip(e, "hipEventElapsedTime"));
}

}  // extern "C"
