// lc_internal.hpp -- internal types of the HIP backend library.
//
// Mirrors the reference's runtime vocabulary (include/lightning_core/core/
// runtime.hpp:11-83): Device, Status, trace events and op kinds, with
// Device::kHIP appended as value 3 so the 4-bit dispatch-trace encoding
// (src/runtime.cpp:703-708) carries it unchanged.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>

#include "lightning_core_hip.h"

namespace lchip {

enum class Status { kSuccess = 0, kNotInitialized, kInvalidValue, kOutOfMemory, kNotSupported, kDriverError, kUnknown };
enum class Device { kCPU = 0, kCUDA = 1, kMetal = 2, kHIP = 3 };

enum class TraceEventType {
  kMallocDevice = 0,
  kFreeDevice,
  kMemcpy,
  kDeviceSynchronize,
  kApplySyncPolicy,
  kGetDeviceCount,
  kIsCudaAvailable,
  kIsMetalAvailable,
  kPreferredDeviceFor,
  kBackendName,
  kOpDispatch
};

enum class TraceOp { kUnknown = 0, kMatMul, kVectorAdd, kMatrixSub, kMatrixDiv, kConv2dNchw, kAttentionForward };

inline lcError_t toLc(Status s) { return static_cast<lcError_t>(static_cast<int>(s)); }
inline Device fromLc(lcDeviceKind d) { return static_cast<Device>(static_cast<int>(d)); }
inline bool validDevice(lcDeviceKind d) { return d >= LC_DEVICE_CPU && d <= LC_DEVICE_HIP; }

// Thread-local last error message (lcGetLastErrorMessage).
void setLastError(const std::string& msg);
const char* lastError();
Status fail(Status st, const std::string& msg);
Status failHip(hipError_t e, const char* what);

#define LC_HIP_TRY(expr)                          \
  do {                                            \
    hipError_t lc_e_ = (expr);                    \
    if (lc_e_ != hipSuccess) {                    \
      return ::lchip::failHip(lc_e_, #expr);      \
    }                                             \
  } while (0)

#define LC_TRY(expr)                              \
  do {                                            \
    ::lchip::Status lc_s_ = (expr);               \
    if (lc_s_ != ::lchip::Status::kSuccess) {     \
      return lc_s_;                               \
    }                                             \
  } while (0)

// ---- runtime trace (ring of 4096 events, off by default) --------------------
constexpr std::size_t kTraceCapacity = 4096;
void traceRecord(TraceEventType type, Status st, std::size_t size_bytes = 0, int d0 = 0, int d1 = 0);
void traceOpDispatch(TraceOp op, Device requested, Device selected, bool fallback, std::size_t workload_hint);
int encodeDispatch(Device requested, Device selected, bool fallback);

// ---- HIP device context --------------------------------------------------------
// Device allocation that grows (1.5x, like the reference's Metal buffers,
// src/attention_metal.mm:150-164) and never shrinks.  Contents are not kept
// across growth.  Freed by reset() or the destructor.
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() { reset(); }
  Status ensure(std::size_t bytes, bool zero = false);
  void reset();
  void* get() const { return ptr_; }
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr_);
  }
  std::size_t size() const { return bytes_; }

 private:
  void* ptr_ = nullptr;
  std::size_t bytes_ = 0;
};

// One context per process for the single visible gfx950 device: one
// non-blocking stream (default priority) that every kernel, copy and event of
// the library uses, and one mutex that serialises host-side use of shared
// buffers (the reference serialises its attention backend the same way,
// src/attention_metal.mm:1855).
// Pinned (page-locked) host staging that grows and never shrinks; allocated
// with hipHostMalloc, which also maps it into the device address space.
// Small calls pack their host operands into it so that one DMA copy replaces
// several pageable ones, or hand its device alias straight to a kernel.
class PinnedBuffer {
 public:
  PinnedBuffer() = default;
  PinnedBuffer(const PinnedBuffer&) = delete;
  PinnedBuffer& operator=(const PinnedBuffer&) = delete;
  ~PinnedBuffer() { reset(); }
  Status ensure(std::size_t bytes);
  void reset();
  void* get() const { return ptr_; }
  // The same bytes as seen by kernels (host writes are visible to a kernel
  // launched after them; kernel writes are visible after a stream sync).
  void* device() const { return dev_; }

 private:
  void* ptr_ = nullptr;
  void* dev_ = nullptr;
  std::size_t bytes_ = 0;
};

struct HipContext {
  std::recursive_mutex mu;
  int device = 0;
  hipStream_t stream = nullptr;
  hipDeviceProp_t props{};
  PinnedBuffer pinned;
  // Stream-K workspace of the fp32 GEMM (partial tiles + ready flags), one
  // slot per workgroup; used by launches on `stream` only, so never shared
  // by two kernels at once.  Each launch publishes with a new epoch
  // (nextStreamKEpoch).  gemm_fail is a pinned, device-mapped word an owner
  // sets when its bounded wait for a partial tile runs out; syncStream turns
  // it into an error.
  DeviceBuffer gemm_part, gemm_flags;
  PinnedBuffer gemm_fail;
  int gemm_epoch = 0;
  // Split-K workspace of the skinny 16-bit GEMM (partials + per-column-tile
  // counters, zero at allocation and after every launch); `stream` only.
  DeviceBuffer skinny_part, skinny_counters;
  // Enqueue-only launches since the stream was last synchronised, per op
  // family (noteEnqueued; syncStream resets both).
  std::size_t matmul_inflight = 0;
  std::size_t attention_inflight = 0;
  // Completion flag of a synchronous small call (waitDoneFlag): the last
  // workgroup of its kernel writes the call's sequence number into done_flag
  // (pinned, device-mapped) after every workgroup's results are visible to
  // the host; done_count (device) counts the finished workgroups and is left
  // at zero by the last one.
  PinnedBuffer done_flag;
  DeviceBuffer done_count;
  unsigned done_seq = 0;
};

bool hipAvailable();
// Returns the context, or nullptr with the status set (kNotSupported when no
// gfx950 device is visible).
HipContext* hipContext(Status* st);

// Upload / download on the context stream (pageable host memory).
Status upload(HipContext* ctx, void* dst, const void* src, std::size_t bytes);
Status download(HipContext* ctx, void* dst, const void* src, std::size_t bytes);
// Synchronises the backend stream, then reports a failure a kernel recorded
// since the last sync (a stream-K wait that ran out) as kDriverError.
Status syncStream(HipContext* ctx);
// The completion flag for the next synchronous small call: allocates it once,
// returns its device alias, the device counter and the call's sequence number.
Status prepareDoneFlag(HipContext* ctx, unsigned** flag_dev, unsigned** count_dev, unsigned* seq);
// Waits for a kernel launched with the flag from prepareDoneFlag to report
// `seq` by spinning on the pinned word (a stream sync costs ~5 us more), then
// does syncStream's bookkeeping.  If the word does not arrive within the
// limit, falls back to syncStream (which reports any launch failure) and
// re-zeroes the counter.
Status waitDoneFlag(HipContext* ctx, unsigned seq);
// Synchronous download of up to four small device results into host memory:
// one copy kernel into the pinned staging raises the completion flag, the
// host waits on it (waitDoneFlag) and copies out.  Returns with the stream
// drained up to that kernel.
struct StagedOut {
  const float* src;  // device
  float* dst;        // host
  std::size_t n;
};
Status stagedDownload(HipContext* ctx, const StagedOut* outs, int count);
// Largest result (floats) worth a staged download: 64 KB came back in 34
// against 65 us per call, 256 KB in 53 against 48 us (the GPU's writes into
// host memory then cost more than a DMA copy).
constexpr std::size_t kStagedDownloadMax = 16384;
// Bookkeeping of enqueue-only launches (no download, no synchronize), as the
// reference's backends cap their in-flight submissions: matmul at 256
// (src/ops/matmul_metal.mm:27, :1864-1878, :1969-1973, :2066-2070),
// attention at 64 (src/attention_metal.mm:26, :1448-1462, :2149-2157).
// Adds `launches` to the op family's count; at the cap the stream is
// synchronised (a device_synchronize trace event with size_bytes = the count,
// detail0 = the op, detail1 = 1) and the count restarts.
constexpr std::size_t kMatMulMaxInflight = 256;
constexpr std::size_t kAttentionMaxInflight = 64;
Status noteEnqueued(HipContext* ctx, TraceOp op, std::size_t launches);
// The epoch for the next stream-K launch over gemm_flags (clears the flags
// on the stream when the counter wraps).
Status nextStreamKEpoch(HipContext* ctx, int* epoch);
// CJ_HIP_STREAMK_SPIN_LIMIT (polls, >= 0), else kern::kStreamKSpinLimit.
int streamKSpinLimit();

inline std::size_t roundUp(std::size_t v, std::size_t m) { return (v + m - 1) / m * m; }

// The device's base architecture ("gfx950"), without the target features
// after ':' -- the arch column of the tune caches.
inline std::string baseArch(const HipContext* ctx) {
  const std::string arch = ctx->props.gcnArchName;
  return arch.substr(0, arch.find(':'));
}

}  // namespace lchip
