/*
 * lightning_core_hip.h -- C ABI of the MI355X (gfx950) backend for Lightning Core.
 *
 * Part 1 restates the reference's frozen C ABI
 * (include/lightning_core/lightning_core.h:1-141 in the reference tree):
 * identical function signatures and struct layouts, with LC_DEVICE_HIP
 * appended to lcDeviceKind after LC_DEVICE_METAL without renumbering.
 *
 * Part 2 adds the compute entry points.  The reference's C ABI has none; each
 * one below is the C form of a C++/pybind entry point of the reference and
 * cites it.  Plain pointers and sizes only.  Host pointers are caller-owned;
 * device buffers are owned by the library (sessions own theirs).
 *
 * Only the "hip" device computes in this library.  Requests for cpu / cuda /
 * metal compute return LC_NOT_SUPPORTED: those devices are served by the
 * reference's own backends, and this library never computes on the CPU.
 * Errors: LC_INVALID_VALUE for null pointers a policy requires or zero sizes;
 * LC_NOT_SUPPORTED when no gfx950 device is visible or a shape / dtype is
 * outside what the kernels handle; LC_DRIVER_ERROR / LC_OUT_OF_MEMORY from HIP.
 * lcGetLastErrorMessage() returns a human-readable reason for the last error.
 */
#ifndef LIGHTNING_CORE_HIP_H
#define LIGHTNING_CORE_HIP_H

#include <stddef.h>
#include <stdint.h>

#define LC_API_VERSION_MAJOR 0
#define LC_API_VERSION_MINOR 6
#define LC_API_VERSION_PATCH 0
#define LC_API_VERSION_STRING "0.6.0-rc0"

#ifdef __cplusplus
extern "C" {
#endif

/* ===== Part 1: the reference's C ABI (lightning_core.h:14-137) ============== */

typedef enum lcError {
  LC_SUCCESS = 0,
  LC_NOT_INITIALIZED,
  LC_INVALID_VALUE,
  LC_OUT_OF_MEMORY,
  LC_NOT_SUPPORTED,
  LC_DRIVER_ERROR,
  LC_UNKNOWN
} lcError_t;

typedef enum lcMemcpyKind {
  LC_MEMCPY_HOST_TO_HOST = 0,
  LC_MEMCPY_HOST_TO_DEVICE,
  LC_MEMCPY_DEVICE_TO_HOST,
  LC_MEMCPY_DEVICE_TO_DEVICE
} lcMemcpyKind;

/* lightning_core.h:31-35, with LC_DEVICE_HIP appended (= 3). */
typedef enum lcDeviceKind {
  LC_DEVICE_CPU = 0,
  LC_DEVICE_CUDA,
  LC_DEVICE_METAL,
  LC_DEVICE_HIP
} lcDeviceKind;

typedef enum lcMemoryModel {
  LC_MEMORY_NATIVE_DEVICE = 0,
  LC_MEMORY_HOST_MANAGED_COMPAT
} lcMemoryModel;

typedef enum lcSyncMode {
  LC_SYNC_AUTO = 0,
  LC_SYNC_ALWAYS,
  LC_SYNC_NEVER
} lcSyncMode;

typedef struct lcSyncPolicy {
  lcSyncMode mode;
  int trace_sync_boundary;
} lcSyncPolicy;

typedef struct lcBackendCapabilities {
  lcDeviceKind device;
  int built;
  int available;
  int compute_surface;
  int memory_surface;
  int sync_surface;
  int profiling_surface;
  int runtime_trace_surface;
  int sync_policy_surface;
  lcMemoryModel memory_model;
} lcBackendCapabilities;

typedef struct lcComputeInterfaceContract {
  int available;
  int op_dispatch_trace_surface;
  const char* driver_tag;
} lcComputeInterfaceContract;

typedef struct lcMemoryInterfaceContract {
  int available;
  int allocator_surface;
  int memcpy_surface;
  lcMemoryModel memory_model;
  const char* driver_tag;
} lcMemoryInterfaceContract;

typedef struct lcSyncInterfaceContract {
  int available;
  int sync_policy_surface;
  int trace_sync_boundary_surface;
  const char* driver_tag;
} lcSyncInterfaceContract;

typedef struct lcProfilerInterfaceContract {
  int available;
  int runtime_trace_surface;
  int op_dispatch_trace_surface;
  size_t trace_capacity;
  const char* driver_tag;
} lcProfilerInterfaceContract;

typedef struct lcBackendInterfaceContract {
  lcDeviceKind device;
  lcBackendCapabilities capabilities;
  lcComputeInterfaceContract compute;
  lcMemoryInterfaceContract memory;
  lcSyncInterfaceContract sync;
  lcProfilerInterfaceContract profiler;
} lcBackendInterfaceContract;

typedef enum lcStructId {
  LC_STRUCT_BACKEND_CAPABILITIES = 1,
  LC_STRUCT_COMPUTE_INTERFACE_CONTRACT = 2,
  LC_STRUCT_MEMORY_INTERFACE_CONTRACT = 3,
  LC_STRUCT_SYNC_INTERFACE_CONTRACT = 4,
  LC_STRUCT_PROFILER_INTERFACE_CONTRACT = 5,
  LC_STRUCT_BACKEND_INTERFACE_CONTRACT = 6
} lcStructId;

/* lightning_core.h:113-137; lcMalloc/lcFree -> hipMalloc/hipFree,
 * lcMemcpy -> hipMemcpy kinds, lcDeviceSynchronize -> backend stream sync. */
lcError_t lcMalloc(void** ptr, size_t size_bytes);
lcError_t lcFree(void* ptr);
lcError_t lcMemcpy(void* dst, const void* src, size_t size_bytes, lcMemcpyKind kind);
lcError_t lcDeviceSynchronize(void);
lcError_t lcGetDeviceCount(int* count);
lcError_t lcGetPreferredDeviceForInference(lcDeviceKind* device);
lcError_t lcGetPreferredDeviceForTraining(lcDeviceKind* device);
int lcIsCudaAvailable(void);
int lcIsMetalAvailable(void);
lcMemoryModel lcGetMemoryModel(void);
const char* lcGetMemoryModelName(lcMemoryModel model);
lcError_t lcSetDefaultSyncPolicy(lcSyncPolicy policy);
lcSyncPolicy lcGetDefaultSyncPolicy(void);
lcError_t lcApplySyncPolicy(lcSyncPolicy policy);
lcError_t lcApplyDefaultSyncPolicy(void);
lcError_t lcGetBackendCapabilities(lcDeviceKind device, lcBackendCapabilities* out_caps);
lcError_t lcGetActiveBackendCapabilities(lcBackendCapabilities* out_caps);
lcError_t lcGetBackendInterfaceContract(lcDeviceKind device, lcBackendInterfaceContract* out_contract);
lcError_t lcGetActiveBackendInterfaceContract(lcBackendInterfaceContract* out_contract);
lcError_t lcGetApiVersion(int* out_major, int* out_minor, int* out_patch);
const char* lcGetApiVersionString(void);
size_t lcGetStructSize(lcStructId struct_id);
int lcCheckStructSize(lcStructId struct_id, size_t observed_size);
const char* lcBackendName(void);
const char* lcGetErrorString(lcError_t error);

/* ===== Part 2: HIP backend additions ======================================== */

/* Parallels lcIsCudaAvailable / lcIsMetalAvailable (lightning_core.h:120-121):
 * 1 when a gfx950 device is visible to HIP. */
int lcIsHipAvailable(void);

/* Human-readable reason for the last non-success status returned on this
 * thread (empty string when none). */
const char* lcGetLastErrorMessage(void);

/* --- runtime trace (reference runtime.hpp:49-83, :222-257) ----------------- */

typedef struct lcRuntimeTraceEvent {
  int type;              /* RuntimeTraceEventType (runtime.hpp:50-62) */
  lcError_t status;
  uint64_t timestamp_ns; /* steady clock */
  size_t size_bytes;     /* bytes, or the op's workload hint for op_dispatch */
  int detail0;           /* op kind for op_dispatch (runtime.hpp:65-73) */
  int detail1;           /* requested | selected << 4 | fallback << 8 */
} lcRuntimeTraceEvent;

void lcSetRuntimeTraceEnabled(int enabled);                                  /* runtime.hpp:223 */
int lcIsRuntimeTraceEnabled(void);                                           /* runtime.hpp:226 */
void lcClearRuntimeTraceEvents(void);                                        /* runtime.hpp:229 */
size_t lcGetRuntimeTraceEvents(lcRuntimeTraceEvent* out, size_t capacity);   /* runtime.hpp:232; returns count */
size_t lcGetRuntimeTraceEventCapacity(void);                                 /* runtime.hpp:235 */
const char* lcRuntimeTraceEventTypeName(int type);                           /* runtime.hpp:238 */
const char* lcRuntimeTraceOpKindName(int op);                                /* runtime.hpp:241 */
int lcEncodeRuntimeTraceDispatchDetail(lcDeviceKind requested, lcDeviceKind selected, int fallback); /* :244 */
int lcDecodeRuntimeTraceDispatchDetail(int encoded, lcDeviceKind* requested, lcDeviceKind* selected,
                                       int* fallback);                       /* runtime.hpp:247-250 */

/* --- compute dtype (new surface: the reference API is fp32-only) ---------- */

typedef enum lcDataType {
  LC_DTYPE_F32 = 0,  /* fp32 storage, fp32 MFMA */
  LC_DTYPE_BF16 = 1, /* bf16 storage, bf16 MFMA, fp32 accumulate */
  LC_DTYPE_F16 = 2   /* fp16 storage, fp16 MFMA, fp32 accumulate */
} lcDataType;

/* --- attention forward ------------------------------------------------------ */

/* AttentionConfig (reference include/lightning_core/core/attention.hpp:9-13). */
typedef struct lcAttentionConfig {
  size_t seq_len;
  size_t head_dim;
  int causal;
} lcAttentionConfig;

/* AttentionIoPolicy (attention.hpp:16-32); defaults from lcAttentionIoPolicyDefault(). */
typedef struct lcAttentionIoPolicy {
  int upload_q;
  int upload_k;
  int upload_v;
  int upload_target;
  int download_out;
  int download_v;
  int synchronize;
  int loss_every;
  float output_scale;
  float output_bias;
  int output_relu;
} lcAttentionIoPolicy;

lcAttentionIoPolicy lcAttentionIoPolicyDefault(void);

/* attentionImplementationName (src/attention.cpp:108-120): "custom-hip-mfma-flash"
 * for LC_DEVICE_HIP when available. */
const char* lcAttentionImplementationName(lcDeviceKind device);

/* attentionForward (src/attention.cpp:127-135): q, k, v, out are host [S, D] fp32. */
lcError_t lcAttentionForward(const float* q, const float* k, const float* v, float* out,
                             const lcAttentionConfig* cfg, lcDeviceKind device);

/* attentionForwardWithPolicy (src/attention.cpp:137-201).  Validation order,
 * workload hint (S*S*D), postprocess out = relu?(out*scale + bias) and the
 * op_dispatch trace follow the reference. */
lcError_t lcAttentionForwardWithPolicy(const float* q, const float* k, const float* v, float* out,
                                       const lcAttentionConfig* cfg, lcDeviceKind device,
                                       const lcAttentionIoPolicy* policy);

/* Batched multi-head attention (new surface; the reference has only the 2-D
 * single-head entry, so this is attentionForwardWithPolicy over batch*heads
 * independent problems).  q, k, v, out: host fp32 [batch, heads, S, D];
 * inputs are rounded to compute_dtype on upload (RNE); fp32 accumulate; out fp32. */
typedef struct lcAttentionBatchedConfig {
  size_t batch;
  size_t heads;
  size_t seq_len;
  size_t head_dim;
  int causal;
  lcDataType compute_dtype;
} lcAttentionBatchedConfig;

lcError_t lcAttentionForwardBatched(const float* q, const float* k, const float* v, float* out,
                                    const lcAttentionBatchedConfig* cfg, lcDeviceKind device,
                                    const lcAttentionIoPolicy* policy);

/* AttentionSession (attention.hpp:86-129, src/attention.cpp:247-283): binds
 * the shape and device and owns persistent device buffers, so upload_q/k/v = 0
 * reuses the resident inputs (upload once, launch only) and download_out = 0
 * leaves the result on the device.  Sessions default to synchronize = 0, as
 * the reference's Metal sessions do (src/attention.cpp:249-253). */
typedef struct lcAttentionSession lcAttentionSession;

lcError_t lcAttentionSessionCreate(const lcAttentionConfig* cfg, lcDeviceKind device, lcAttentionSession** out);
lcError_t lcAttentionSessionCreateBatched(const lcAttentionBatchedConfig* cfg, lcDeviceKind device,
                                          lcAttentionSession** out);
lcError_t lcAttentionSessionDestroy(lcAttentionSession* session);
lcError_t lcAttentionSessionSetDefaultPolicy(lcAttentionSession* session, const lcAttentionIoPolicy* policy);
lcError_t lcAttentionSessionGetDefaultPolicy(const lcAttentionSession* session, lcAttentionIoPolicy* out);
lcError_t lcAttentionSessionForward(lcAttentionSession* session, const float* q, const float* k, const float* v,
                                    float* out);
lcError_t lcAttentionSessionForwardWithPolicy(lcAttentionSession* session, const float* q, const float* k,
                                              const float* v, float* out, const lcAttentionIoPolicy* policy);
/* Launch-only repeat of the resident forward (no uploads, no download), then
 * a stream synchronisation: the attention analogue of
 * MatMulMetalResidentSession::runBatchSyncCachedNoDownload (ops.hpp:1371-1373). */
lcError_t lcAttentionSessionRunCached(lcAttentionSession* session, size_t repeat_count);

/* Attention train step, fp32, one head [S, D] (the reference's dV-only SGD
 * step): out = attention(q, k, v) (no postprocess), loss = mean((out -
 * target)^2), v -= learning_rate * P^T . 2 (out - target) / (S*D).  v is
 * in/out: with download_v the updated V is copied back into it.  Null
 * pointers, zero dims or learning_rate <= 0 -> LC_INVALID_VALUE regardless of
 * the policy (src/attention.cpp:229-232).  loss_out may be NULL (no loss).
 * attentionTrainStep (src/attention.cpp:203-214). */
lcError_t lcAttentionTrainStep(const float* q, const float* k, float* v, const float* target, float* out,
                               float learning_rate, const lcAttentionConfig* cfg, lcDeviceKind device,
                               float* loss_out);
/* attentionTrainStepWithPolicy (src/attention.cpp:217-244): upload_q/k/v/
 * target = 0 reuse the backend-global resident tensors, download_out /
 * download_v / synchronize as for the forward. */
lcError_t lcAttentionTrainStepWithPolicy(const float* q, const float* k, float* v, const float* target, float* out,
                                         float learning_rate, const lcAttentionConfig* cfg, lcDeviceKind device,
                                         float* loss_out, const lcAttentionIoPolicy* policy);
/* AttentionSession::trainStep / trainStepWithPolicy (src/attention.cpp:
 * 285-343): on the session's own resident tensors; with loss_out, the loss is
 * measured every loss_every steps (0 = shape-aware default, :12-39) and the
 * last measured value is returned in between, when a step downloads nothing
 * it then does not block. */
lcError_t lcAttentionSessionTrainStep(lcAttentionSession* session, const float* q, const float* k, float* v,
                                      const float* target, float* out, float learning_rate, float* loss_out);
lcError_t lcAttentionSessionTrainStepWithPolicy(lcAttentionSession* session, const float* q, const float* k,
                                                float* v, const float* target, float* out, float learning_rate,
                                                float* loss_out, const lcAttentionIoPolicy* policy);

/* Launch-only repeat of the session's resident train step (no uploads, no
 * downloads, no loss; V updated in place on the device each step), then a
 * stream synchronisation.  The loop of the reference's training benchmark on
 * its resident fast path (benchmarks/bench_attention.cpp:248-269, which calls
 * AttentionSession::trainStep per step), run in C; the train-step analogue of
 * lcAttentionSessionRunCached.  Needs q, k, v and target resident (a step that
 * uploaded them); learning_rate <= 0 -> LC_INVALID_VALUE. */
lcError_t lcAttentionSessionTrainRunCached(lcAttentionSession* session, float learning_rate, size_t repeat_count);

/* --- matmul ------------------------------------------------------------------ */

/* MatMulIoPolicy (reference include/lightning_core/core/ops/policy.hpp:8-13). */
typedef struct lcMatMulIoPolicy {
  int upload_a;
  int upload_b;
  int download_out;
  int synchronize;
} lcMatMulIoPolicy;

lcMatMulIoPolicy lcMatMulIoPolicyDefault(void);

/* ops::matMul<float> (ops.hpp:195-205): host row-major fp32 A[M,K], B[K,N], C[M,N]. */
lcError_t lcMatMul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n, lcDeviceKind device);

/* ops::matMulWithPolicy<float> (ops.hpp:354-459).  Null a/b/out are allowed
 * when the policy does not upload/download them; then the backend's resident
 * buffers (last uploaded) are used, as the reference's global Metal context
 * does (matmul_metal.mm:1836-1937). */
lcError_t lcMatMulWithPolicy(const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                             lcDeviceKind device, const lcMatMulIoPolicy* policy);

/* detail::matMulMetalWithPolicyBatched (matmul_metal.mm:1939-2075 /
 * ops_backend.hpp:254-265): `repeat_count` launches in one submission. */
lcError_t lcMatMulWithPolicyBatched(const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                                    lcDeviceKind device, const lcMatMulIoPolicy* policy, size_t repeat_count);

/* matMulMetalResetTuning (ops_backend.hpp:295): clears the gfx950 tune cache. */
lcError_t lcMatMulResetTuning(void);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc).  A
 * synchronous call on the library's own stream (it clears a failure word with
 * hipMemsetAsync, copies it back and synchronises before returning), so it
 * must not be called while a stream capture is active.  out = a . b in fp32
 * with the kernels of lcMatMul, on
 * device-resident row-major a [m, k], b [k, n], out [m, n]; every other byte
 * the kernels touch (stream-K partial tiles and flags, zero-padded copies of
 * an operand whose dims are not multiples of 64 or whose base is not 16-byte
 * aligned) lives in a fixed 32 MiB static device array that each GPU holds
 * until the process ends.  Allocates nothing; synchronises the backend stream
 * before returning.  Padded copies beyond the array (28 MiB for both) ->
 * LC_NOT_SUPPORTED; pointers HIP does not know as device memory ->
 * LC_INVALID_VALUE.  All calls on one GPU share the array: the library
 * serialises its own callers, calls that overlap on one GPU otherwise race. */
lcError_t lcMatMulDeviceNoAlloc(const float* a, const float* b, float* out, size_t m, size_t k, size_t n);

/* MatMulMetalResidentSession<T> (ops.hpp:1339-1379), with session-owned
 * device buffers and a compute dtype (fp32 host data is rounded to bf16/fp16
 * once at upload, like the reference's fp16 resident batch path,
 * matmul_metal.mm:1421-1524).  Output is fp32. */
typedef struct lcMatMulResidentSession lcMatMulResidentSession;

lcError_t lcMatMulResidentSessionCreate(size_t m, size_t k, size_t n, lcDataType compute_dtype,
                                        lcMatMulResidentSession** out);
lcError_t lcMatMulResidentSessionDestroy(lcMatMulResidentSession* s);
lcError_t lcMatMulResidentSessionStart(lcMatMulResidentSession* s, const float* a, const float* b, float* out);  /* :1347 */
lcError_t lcMatMulResidentSessionRun(lcMatMulResidentSession* s, const float* a, const float* b, float* out);    /* :1351 */
lcError_t lcMatMulResidentSessionFinish(lcMatMulResidentSession* s, const float* a, const float* b, float* out); /* :1355 */
lcError_t lcMatMulResidentSessionSync(lcMatMulResidentSession* s, const float* a, const float* b, float* out);   /* :1359 */
lcError_t lcMatMulResidentSessionRunBatchSync(lcMatMulResidentSession* s, const float* a, const float* b,
                                              float* out, size_t repeat_count);                                  /* :1363 */
lcError_t lcMatMulResidentSessionRunBatchSyncNoDownload(lcMatMulResidentSession* s, const float* a,
                                                        const float* b, float* out, size_t repeat_count);        /* :1367 */
lcError_t lcMatMulResidentSessionRunBatchSyncCachedNoDownload(lcMatMulResidentSession* s, size_t repeat_count); /* :1371 */
/* Measurement helpers, no reference counterpart (the roofline timing of a
 * single kernel).  TimeLaunches: `count` launch-only GEMMs on the resident
 * inputs, back to back on the backend stream with a hipEvent pair around each
 * launch, then a sync; ms_out[i] = launch i's event-measured duration.
 * KernelName: "<tune-cache variant> <kernel function>" of the GEMM the
 * session's shape runs (e.g. "half_w4h_256x256 gemm_half_tn_w4h_kernel"). */
lcError_t lcMatMulResidentSessionTimeLaunches(lcMatMulResidentSession* s, size_t count, float* ms_out);
lcError_t lcMatMulResidentSessionKernelName(lcMatMulResidentSession* s, char* buf, size_t cap);

/* --- conv2d and the integrated conv -> attention pipeline -------------------- */

/* ops::conv2dNchw<float> (ops.hpp:855-1213): x [B,C,H,W], w [OC,C,KH,KW],
 * bias [OC] or NULL, out [B,OC,OH,OW]; implicit GEMM on the GPU with the
 * bias / ReLU epilogue fused. */
lcError_t lcConv2dNchw(const float* x, const float* w, const float* bias, float* out, size_t batch,
                       size_t in_channels, size_t in_h, size_t in_w, size_t out_channels, size_t kernel_h,
                       size_t kernel_w, size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w,
                       lcDeviceKind device, int apply_relu);

/* api.conv_attention_torchstrong_nchw_into (bind_integrated.cpp:614-730,
 * eager mode): conv2d + ReLU, Q/K/V = consecutive seq_len*head_dim slices of
 * the flat NCHW output (repeated when short, QkvPackRepeat), single-head
 * non-causal attention; out [seq_len, head_dim].  All stages stay on the GPU. */
lcError_t lcConvAttentionTorchstrongNchw(const float* x, const float* w, const float* bias, float* out,
                                         size_t batch, size_t in_channels, size_t in_h, size_t in_w,
                                         size_t out_channels, size_t kernel_h, size_t kernel_w, size_t seq_len,
                                         size_t head_dim, size_t stride_h, size_t stride_w, size_t pad_h,
                                         size_t pad_w, lcDeviceKind device);

/* The same call in graph mode (convAttentionTorchstrongNchwIntoGraph,
 * bind_integrated.cpp:745-837): 3x3 weights only (else LC_NOT_SUPPORTED with
 * the reference's message); one plan per key (geometry, seq_len, head_dim,
 * has_bias), here a HIP graph captured on the first call and replayed after.
 * Results equal the eager call's.  Clear drops every plan (syncs first). */
lcError_t lcConvAttentionTorchstrongNchwGraph(const float* x, const float* w, const float* bias, float* out,
                                              size_t batch, size_t in_channels, size_t in_h, size_t in_w,
                                              size_t out_channels, size_t kernel_h, size_t kernel_w, size_t seq_len,
                                              size_t head_dim, size_t stride_h, size_t stride_w, size_t pad_h,
                                              size_t pad_w, lcDeviceKind device);
lcError_t lcConvAttentionGraphCacheClear(void);
size_t lcConvAttentionGraphCacheSize(void);

/* ViT-style block (new composition of the reference's conv2dNchw, matMul and
 * attentionForward): patch-embed conv (kernel = stride = patch, no padding,
 * no bias) + ReLU -> tokens [B, T, E] -> QKV = tokens . w_qkv [E, 3E] split in
 * timm (B, T, 3, H, Dh) order -> per-head non-causal attention -> concat ->
 * . w_o [E, E].  x [B, C, H, W], w_conv [E, C, P, P], out [B, T, E] fp32. */
typedef struct lcVitBlockConfig {
  size_t batch;
  size_t in_channels;
  size_t image_h;
  size_t image_w;
  size_t patch;
  size_t embed;
  size_t heads;
  lcDataType compute_dtype;
} lcVitBlockConfig;

typedef struct lcVitBlockSession lcVitBlockSession;

lcError_t lcVitBlockSessionCreate(const lcVitBlockConfig* cfg, lcDeviceKind device, lcVitBlockSession** out);
lcError_t lcVitBlockSessionDestroy(lcVitBlockSession* s);
/* Uploads (and converts) the weights; they stay resident. */
lcError_t lcVitBlockSessionSetWeights(lcVitBlockSession* s, const float* w_conv, const float* w_qkv,
                                      const float* w_o);
/* One forward: x uploaded when non-NULL (else the resident input is reused),
 * out downloaded when non-NULL; synchronises when out is non-NULL. */
lcError_t lcVitBlockSessionForward(lcVitBlockSession* s, const float* x, float* out);
/* Launch-only repeat over the resident input, then a stream synchronisation. */
lcError_t lcVitBlockSessionRunCached(lcVitBlockSession* s, size_t repeat_count);

lcError_t lcVitBlockForward(const float* x, const float* w_conv, const float* w_qkv, const float* w_o, float* out,
                            const lcVitBlockConfig* cfg, lcDeviceKind device);

/* --- device info and timing on the backend stream ---------------------------- */

typedef struct lcHipDeviceInfo {
  char name[128];
  char gcn_arch[64];
  int compute_units;
  int max_clock_khz;
  size_t total_memory_bytes;
  size_t l2_cache_bytes;
} lcHipDeviceInfo;

lcError_t lcHipGetDeviceInfo(lcHipDeviceInfo* out);

/* HIP events recorded on the backend stream (the stream every kernel of this
 * library is launched on); Stop synchronises on the stop event and returns
 * the elapsed milliseconds. */
typedef struct lcHipTimer lcHipTimer;
lcError_t lcHipTimerCreate(lcHipTimer** out);
lcError_t lcHipTimerDestroy(lcHipTimer* t);
lcError_t lcHipTimerStart(lcHipTimer* t);
lcError_t lcHipTimerStop(lcHipTimer* t, float* elapsed_ms);

/* The gfx950 matmul tune cache: the reference's file convention
 * (src/ops/matmul_metal.mm:133-139, :416-517) with rows re-keyed for gfx950
 * (m,k,n,dtype,arch,kernel variant).  It is also loaded implicitly on the
 * first matmul (CJ_MATMUL_TUNE_CACHE_FILE, else
 * .lightning_core_matmul_tune_cache.csv in the working directory) and
 * rewritten when a new shape is tuned; versions 1 and 2 are read, 2 written.
 * Load makes `path` the cache file; a header of another kind or version
 * clears the table and returns LC_INVALID_VALUE. */
lcError_t lcHipTuneCacheSave(const char* path);
lcError_t lcHipTuneCacheLoad(const char* path);
size_t lcHipTuneCacheSize(void);

/* The attention tune cache (src/attention_metal.mm:184-336, same layout:
 * F,seq,dim,causal,resident_hint,sync_hint,mode and T rows with compute_loss);
 * the mode is the gfx950 fp32 kernel's split count (1, 2, 4, 8).  Implicit
 * file: CJ_ATTN_TUNE_CACHE_FILE, else .lightning_core_attn_tune_cache.csv. */
lcError_t lcHipAttentionTuneCacheSave(const char* path);
lcError_t lcHipAttentionTuneCacheLoad(const char* path);
lcError_t lcHipAttentionResetTuning(void);
size_t lcHipAttentionTuneCacheSize(void);

/* runtime::preloadRuntimeProfileEnv (core/runtime.hpp:193,
 * src/runtime.cpp:101-168, :421-423): imports CJ_* variables from the runtime
 * profile file once per process (CJ_RUNTIME_PROFILE_ENV_FILE or the
 * reference's cwd-relative candidates; CJ_RUNTIME_PROFILE_AUTOLOAD=0 skips). */
void lcPreloadRuntimeProfileEnv(void);

/* --- graph IR on hip (reference lightning_core::graph::GraphIR,
 * include/lightning_core/core/graph.hpp; its Python class GraphIR,
 * python/bindings/bind_graph.cpp:340-906) ------------------------------------
 * The nine operators ("matmul", "vector_add", "matrix_sub", "matrix_div",
 * "attention_forward", "conv2d_nchw3x3", "conv2d_nchw3x3s1p1",
 * "qkv_pack_repeat", "relu") with the reference's schemas plus a hip column,
 * its validation passes and reason codes, the capability-scored planner with
 * sync boundaries and plan cache, the fusion report with cost model v1/v2,
 * and an executor that runs every node on the GPU.  Reporting calls keep a
 * JSON report in the graph (the report of the last call on that graph),
 * copied out by lcGraphReport; calls on one graph are serialised.  Tensor
 * dtype: 0 float32, 1 float64; layout: 0 contiguous, 1 strided.  No
 * counterpart in the reference C ABI (its graph is C++ / pybind only). */
typedef struct lcGraph lcGraph;

/* GraphPlannerOptions (graph.hpp:462-499); sync_mode 0 auto, 1 always,
 * 2 never; NULL strings mean the reference defaults
 * ("conv,matmul,attention,attention_qkv", "auto"). */
typedef struct lcGraphPlannerOptions {
  lcDeviceKind preferred_device;
  int sync_mode;
  int trace_sync_boundary;
  int group_by_backend_capability;
  int separate_fallback_segments;
  int insert_sync_on_device_change;
  int enable_fusion_v1;
  int enable_fusion_pass_conv;
  int enable_fusion_pass_matmul;
  int enable_fusion_pass_attention;
  int enable_fusion_pass_attention_qkv;
  const char* fusion_pass_order;
  int enable_fusion_cost_model_v1;
  int enable_fusion_cost_model_v2;
  int enable_plan_cache;
  const char* cost_profile_signature;
  double fusion_cost_min_speedup;
  double cost_launch_overhead_ns;
  double cost_transfer_overhead_ns;
  double cost_sync_boundary_ns;
  double cost_elementwise_per_element_ns;
  double cost_matmul_per_mac_ns;
  double cost_conv_per_mac_ns;
  double planner_cost_weight_compute;
  double planner_cost_weight_boundary;
  double planner_cost_weight_preference;
} lcGraphPlannerOptions;

/* The reference defaults with preferred_device = LC_DEVICE_HIP. */
lcGraphPlannerOptions lcGraphPlannerOptionsDefault(void);
lcError_t lcGraphCreate(lcGraph** out);
lcError_t lcGraphDestroy(lcGraph* g);
/* GraphIR::addTensorSpec (graph.hpp:620-640): every dimension > 0. */
lcError_t lcGraphAddTensor(lcGraph* g, const int64_t* shape, size_t rank, int dtype, int layout, const char* name,
                           int constant, size_t* out_id);
/* GraphIR::addNode (graph.hpp:642-684): an unknown op is LC_NOT_SUPPORTED;
 * wrong arity, tensor ids out of range or control dependencies on later
 * nodes are LC_INVALID_VALUE.  Attributes as parallel arrays. */
lcError_t lcGraphAddNode(lcGraph* g, const char* op, const size_t* inputs, size_t n_inputs, const size_t* outputs,
                         size_t n_outputs, const size_t* control_deps, size_t n_control_deps, const char* name,
                         const char* const* attr_keys, const int64_t* attr_values, size_t n_attrs);
lcError_t lcGraphCounts(lcGraph* g, size_t* num_tensors, size_t* num_nodes);
/* GraphIR::planCacheStats / clearPlanCache (graph.hpp:1722-1738). */
lcError_t lcGraphPlanCacheStats(lcGraph* g, size_t* hits, size_t* misses);
lcError_t lcGraphClearPlanCache(lcGraph* g);
/* Copies the report of the last reporting call on g: json == NULL (or
 * cap == 0) only sets *needed (bytes including the NUL); a smaller buffer is
 * LC_INVALID_VALUE.  Has no other effect. */
lcError_t lcGraphReport(lcGraph* g, char* json, size_t cap, size_t* needed);
/* Report {"tensors": [...], "nodes": [...]} (bind_graph.cpp:408-421). */
lcError_t lcGraphDescribe(lcGraph* g);
/* graph_registry_schemas (bind_graph.cpp:323-330) as a JSON list. */
lcError_t lcGraphRegistry(char* json, size_t cap, size_t* needed);
/* validateWithReport (graph.hpp:690-1062): report {"ok", "status", "issues"},
 * written whatever the outcome; returns the validation status. */
lcError_t lcGraphValidate(lcGraph* g);
/* planForDevice (graph.hpp:1064-1079): report = the plan steps. */
lcError_t lcGraphPlanForDevice(lcGraph* g, lcDeviceKind preferred_device);
/* plan_groups (bind_graph.cpp:440-508): {"groups", "steps", "summary"}. */
lcError_t lcGraphPlanGroups(lcGraph* g, const lcGraphPlannerOptions* options);
/* planSummary (graph.hpp:1325-1361): {"summary", "groups", "steps"}. */
lcError_t lcGraphPlanSummary(lcGraph* g, const lcGraphPlannerOptions* options);
/* fusionReport (graph.hpp:1392-1707): the fusion decisions as a list. */
lcError_t lcGraphFusionReport(lcGraph* g, const lcGraphPlannerOptions* options);
/* executeF32 (graph.hpp:1364-1372) on hip: feeds (host fp32, feed_sizes
 * elements each, equal to the tensor's element count) are uploaded once;
 * every node runs on the GPU in plan order with the reference's fusion walk
 * (graph.hpp:3586-3840); the requested tensors are copied to `outputs` after
 * one sync.  Report {"groups", "steps", "summary"}.  A plan that puts any
 * node on another device (preferred_device "cpu", float64 tensors) is
 * LC_NOT_SUPPORTED naming the node, before any launch: this backend has no
 * CPU compute path.  A tensor that is neither fed nor produced, when read or
 * requested, is LC_INVALID_VALUE. */
lcError_t lcGraphExecuteF32(lcGraph* g, const lcGraphPlannerOptions* options, const size_t* feed_ids,
                            const float* const* feeds, const size_t* feed_sizes, size_t n_feeds,
                            const size_t* output_ids, float* const* outputs, size_t n_outputs);

#ifdef __cplusplus
}
#endif

#endif /* LIGHTNING_CORE_HIP_H */
