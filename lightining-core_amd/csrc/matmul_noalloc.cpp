// matmul_noalloc.cpp -- the fp32 GEMM entry point that allocates nothing.
//
// lcMatMulDeviceNoAlloc computes C = A . B like lcMatMul, with the same
// kernels (gemm_f32_lds_kernel, whole tiles or stream-K), for callers that
// cannot allocate device memory: tight serving loops and harnesses that
// forbid hipMalloc.  It is a synchronous call on the library's own stream:
// it clears the failure word (hipMemsetAsync), launches, copies the failure
// word to the host and synchronises that stream before returning, so it must
// not be called while a stream capture is active (it records nothing into a
// caller's graph).  The caller passes device-resident A, B and C; every other
// byte the kernels touch lives in `scratch`, a file-scope device array of
// kScratchBytes that each GPU holds until the process ends:
//
//   [0, 4 MiB)          stream-K partial tiles (256 workgroups x 64 x 64 fp32)
//   [4 MiB, +1 KiB)     stream-K ready flags (256 ints)
//   [4 MiB + 1 KiB, +4) the launch's failure word
//   [kOperandOffset, ..) zero-padded copies of A and/or B, when M, K or N is
//                        not a multiple of 64 (the kernel reads whole tiles)
//
// Host code never passes `scratch` itself to a kernel or a copy: in host code
// the name stands for a host-side shadow, not a device address.  The device
// address is taken once per device with hipGetSymbolAddress (the device
// current) and kept per device.  All calls on one GPU share that GPU's array,
// which keeps the last call's contents: the kernel clears the flags it
// consumed and each launch publishes with a new epoch (so a flag a timed-out
// launch left set is never taken for ready), and after a launch whose wait
// ran out the flags are zeroed before the call returns; the failure word is
// cleared on the stream before each launch.  Calls hold the library's context
// mutex, so calls from threads of one process are serialised; calls that
// overlap on one GPU from different processes or outside the library race.
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>

#include "ops_internal.hpp"

namespace lchip {
namespace {

constexpr std::size_t kScratchBytes = std::size_t(32) << 20;
constexpr int kMaxGroups = 256;
constexpr std::size_t kPartBytes = std::size_t(kMaxGroups) * 4096 * sizeof(float);
constexpr std::size_t kFlagsOffset = kPartBytes;
constexpr std::size_t kFailOffset = kFlagsOffset + kMaxGroups * sizeof(int);
constexpr std::size_t kOperandOffset = kPartBytes + 64 * 1024;  // 256-byte aligned
constexpr std::size_t kOperandBytes = kScratchBytes - kOperandOffset;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct ScratchSlot {
  unsigned char* ptr = nullptr;  // device address of `scratch` on this device
  int epoch = 0;                 // last stream-K epoch used on these flags
};

std::mutex g_slot_mu;
ScratchSlot g_slots[kMaxDevices];

// The device address of this device's `scratch`, taken once (set-up).
Status scratchFor(int device, ScratchSlot** out) {
  if (device < 0 || device >= kMaxDevices) {
    return fail(Status::kNotSupported, "matmul no-alloc: device index out of range");
  }
  std::lock_guard<std::mutex> lock(g_slot_mu);
  ScratchSlot& s = g_slots[device];
  if (s.ptr == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      return failHip(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    }
    s.ptr = static_cast<unsigned char*>(p);
  }
  *out = &s;
  return Status::kSuccess;
}

std::size_t paddedBytes(std::size_t rows, std::size_t cols) {
  return roundUp(rows, 64) * roundUp(cols, 64) * sizeof(float);
}

// True when HIP knows `p` as device (or managed) memory; a kernel handed a
// host pointer would fault.  The query allocates nothing; a failed query's
// sticky error is cleared so a later launch status is not mistaken for it.
bool isDeviceMemory(const void* p) {
  hipPointerAttribute_t attr{};
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

}  // namespace

Status matmulDeviceNoAlloc(const float* a, const float* b, float* c, std::size_t m, std::size_t k, std::size_t n) {
  if (a == nullptr || b == nullptr || c == nullptr || m == 0 || k == 0 || n == 0) {
    return fail(Status::kInvalidValue, "matmul no-alloc: null pointer or zero dimension");
  }
  if (m > (1u << 30) || k > (1u << 30) || n > (1u << 30) || 64 * roundUp(k, 64) * 4 >= (std::size_t(1) << 31) ||
      64 * roundUp(n, 64) * 4 >= (std::size_t(1) << 31)) {
    return fail(Status::kNotSupported, "matmul no-alloc: shape too large");
  }
  // The kernel reads whole 64-wide tiles with 16-byte loads: an operand is
  // copied (zero padded) into the scratch unless its dims are multiples of 64
  // and its base is 16-byte aligned.
  const bool pad_a = (m % 64) != 0 || (k % 64) != 0 || reinterpret_cast<std::uintptr_t>(a) % 16 != 0;
  const bool pad_b = (k % 64) != 0 || (n % 64) != 0 || reinterpret_cast<std::uintptr_t>(b) % 16 != 0;
  const std::size_t a_bytes = pad_a ? paddedBytes(m, k) : 0;
  const std::size_t b_bytes = pad_b ? paddedBytes(k, n) : 0;
  if (roundUp(a_bytes, 256) + b_bytes > kOperandBytes) {
    return fail(Status::kNotSupported,
                "matmul no-alloc: the zero-padded operand copies (" + std::to_string(a_bytes + b_bytes) +
                    " bytes; M, K or N not a multiple of 64) exceed the fixed scratch of " +
                    std::to_string(kOperandBytes) + " bytes");
  }
  HipContext* ctx = nullptr;
  LC_TRY(requireHip(LC_DEVICE_HIP, "matmul no-alloc", &ctx));
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  if (!isDeviceMemory(a) || !isDeviceMemory(b) || !isDeviceMemory(c)) {
    return fail(Status::kInvalidValue, "matmul no-alloc: a, b and out must be device memory");
  }
  ScratchSlot* slot = nullptr;
  LC_TRY(scratchFor(ctx->device, &slot));
  unsigned char* base = slot->ptr;

  const float* A = a;
  const float* B = b;
  const int kp = static_cast<int>(roundUp(k, 64));
  const int np = static_cast<int>(roundUp(n, 64));
  if (pad_a) {
    float* ap = reinterpret_cast<float*>(base + kOperandOffset);
    LC_HIP_TRY(kern::padCopyF32(a, ap, static_cast<int>(m), static_cast<int>(k), k, static_cast<int>(roundUp(m, 64)),
                                kp, ctx->stream));
    A = ap;
  }
  if (pad_b) {
    float* bp = reinterpret_cast<float*>(base + kOperandOffset + roundUp(a_bytes, 256));
    LC_HIP_TRY(kern::padCopyF32(b, bp, static_cast<int>(k), static_cast<int>(n), n, kp, np, ctx->stream));
    B = bp;
  }
  const int groups = std::min(kMaxGroups, ctx->props.multiProcessorCount > 0 ? ctx->props.multiProcessorCount
                                                                             : kMaxGroups);
  int* fail_word = reinterpret_cast<int*>(base + kFailOffset);
  LC_HIP_TRY(hipMemsetAsync(fail_word, 0, sizeof(int), ctx->stream));
  if (slot->epoch >= (1 << 30)) {
    LC_HIP_TRY(hipMemsetAsync(base + kFlagsOffset, 0, kMaxGroups * sizeof(int), ctx->stream));
    slot->epoch = 0;
  }
  kern::StreamKSync sync{reinterpret_cast<float*>(base), reinterpret_cast<int*>(base + kFlagsOffset), fail_word,
                         ++slot->epoch, streamKSpinLimit()};
  traceOpDispatch(TraceOp::kMatMul, Device::kHIP, Device::kHIP, false, m * k * n);
  // unpadded operands have k == kp and n == np, so the leading dims agree
  LC_HIP_TRY(kern::gemmF32Padded(A, B, c, static_cast<int>(m), static_cast<int>(n), kp, kp, np, static_cast<int>(n),
                                 sync, groups, kern::GemmF32Variant::kAuto, ctx->stream));
  int failed = 0;
  LC_HIP_TRY(hipMemcpyAsync(&failed, fail_word, sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
  LC_TRY(syncStream(ctx));
  if (failed != 0) {
    // The kernel has completed, so no publisher is still running: zero the
    // flags a late publisher may have set, so no later launch can meet them.
    LC_HIP_TRY(hipMemsetAsync(base + kFlagsOffset, 0, kMaxGroups * sizeof(int), ctx->stream));
    LC_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return fail(Status::kDriverError,
                "matmul no-alloc: a stream-K workgroup's bounded wait for a partial tile ran out "
                "(CJ_HIP_STREAMK_SPIN_LIMIT); the result is invalid");
  }
  return Status::kSuccess;
}

}  // namespace lchip

extern "C" lcError_t lcMatMulDeviceNoAlloc(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) {
  return lchip::toLc(lchip::matmulDeviceNoAlloc(a, b, out, m, k, n));
}
