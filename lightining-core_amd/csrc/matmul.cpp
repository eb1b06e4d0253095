// matmul.cpp -- matmul front-end for the "hip" device.
//
// Mirrors ops::matMulWithPolicy<float> (reference include/lightning_core/
// core/ops.hpp:354-459) and MatMulMetalResidentSession<T> (:1339-1379):
//   * validation: (upload_a && !a) || (upload_b && !b) || (download_out &&
//     !out) || any zero dim -> kInvalidValue (:367-370);
//   * workload hint m*k*n in the op_dispatch trace (:366);
//   * resident protocol start (upload, no download, no sync), run (launch
//     only), finish (download + sync), sync (sync only), and the batched
//     launch-only forms (:207-352, policy.hpp:37-71);
//   * buffers of the policy-level API live in one backend-global slot, as the
//     reference's Metal context (matmul_metal.mm:1836-1937); sessions own
//     their own buffers instead.
// 16-bit compute rounds the fp32 host data once at upload (RNE) and lays B out
// K-contiguous (transposed), the layout the MFMA GEMM reads.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iterator>
#include <string>
#include <vector>

#include "ops_internal.hpp"
#include "tune.hpp"

namespace lchip {

namespace {

Status uploadA(HipContext* ctx, MatMulResident& r, const float* a) {
  if (!isHalf(r.dtype)) {
    // fp32: A [roundup(M, 64), roundup(K, 64)], zero pads
    const std::size_t mp = roundUp(r.m, kern::kF32GemmBM);
    const std::size_t kp = roundUp(r.k, kern::kF32GemmBK);
    LC_TRY(r.stage.ensure(r.m * r.k * sizeof(float)));
    LC_TRY(r.a.ensure(mp * kp * sizeof(float)));
    LC_TRY(upload(ctx, r.stage.get(), a, r.m * r.k * sizeof(float)));
    const hipError_t e = kern::padCopyF32(r.stage.as<float>(), r.a.as<float>(), static_cast<int>(r.m),
                                          static_cast<int>(r.k), r.k, static_cast<int>(mp), static_cast<int>(kp),
                                          ctx->stream);
    return e == hipSuccess ? Status::kSuccess : failHip(e, "matmul upload padding (A)");
  }
  const std::size_t mp = roundUp(r.m, kern::kHalfGemmBM);
  const std::size_t kp = roundUp(r.k, kern::kHalfGemmBK);
  LC_TRY(r.stage.ensure(r.m * r.k * sizeof(float)));
  LC_TRY(r.a.ensure(mp * kp * sizeof(uint16_t)));
  LC_TRY(upload(ctx, r.stage.get(), a, r.m * r.k * sizeof(float)));
  const hipError_t e = kern::convertPad(r.stage.as<float>(), r.a.as<uint16_t>(), 1, static_cast<int>(r.m),
                                        static_cast<int>(r.k), r.k, static_cast<int>(mp), static_cast<int>(kp), 0, 0,
                                        halfOf(r.dtype), ctx->stream);
  return e == hipSuccess ? Status::kSuccess : failHip(e, "matmul upload conversion (A)");
}

Status uploadB(HipContext* ctx, MatMulResident& r, const float* b) {
  if (!isHalf(r.dtype)) {
    // fp32: B [roundup(K, 64), roundup(N, 64)], zero pads
    const std::size_t kp = roundUp(r.k, kern::kF32GemmBK);
    const std::size_t np = roundUp(r.n, kern::kF32GemmBN);
    LC_TRY(r.stage.ensure(r.k * r.n * sizeof(float)));
    LC_TRY(r.b.ensure(kp * np * sizeof(float)));
    LC_TRY(upload(ctx, r.stage.get(), b, r.k * r.n * sizeof(float)));
    const hipError_t e = kern::padCopyF32(r.stage.as<float>(), r.b.as<float>(), static_cast<int>(r.k),
                                          static_cast<int>(r.n), r.n, static_cast<int>(kp), static_cast<int>(np),
                                          ctx->stream);
    return e == hipSuccess ? Status::kSuccess : failHip(e, "matmul upload padding (B)");
  }
  const std::size_t np = roundUp(r.n, kern::kHalfGemmBN);
  const std::size_t kp = roundUp(r.k, kern::kHalfGemmBK);
  LC_TRY(r.stage.ensure(r.k * r.n * sizeof(float)));
  LC_TRY(r.b.ensure(np * kp * sizeof(uint16_t)));
  LC_TRY(upload(ctx, r.stage.get(), b, r.k * r.n * sizeof(float)));
  // B [K, N] -> Bt [N_pad, K_pad]
  const hipError_t e = kern::convertTransposePad(r.stage.as<float>(), r.b.as<uint16_t>(), 1, static_cast<int>(r.k),
                                                 static_cast<int>(r.n), r.n, static_cast<int>(kp),
                                                 static_cast<int>(np), 0, 0, halfOf(r.dtype), ctx->stream);
  return e == hipSuccess ? Status::kSuccess : failHip(e, "matmul upload conversion (B)");
}

// Tune-cache names of the GEMM variants and the configuration each stands
// for (block tile M x N x K, waves, K-split of a stage between wave groups).
struct VariantInfo {
  int variant;
  const char* name;
  int tile_m, tile_n, tile_k, waves, split_k;
  const char* hip_kernel;  // the __global__ function that runs it
};

constexpr VariantInfo kF32Variants[] = {
    {static_cast<int>(kern::GemmF32Variant::kDataParallel), "f32_dp_64x64x64", 64, 64, 64, 8, 2,
     "gemm_f32_lds_kernel"},
    {static_cast<int>(kern::GemmF32Variant::kStreamK), "f32_streamk_64x64x64", 64, 64, 64, 8, 2,
     "gemm_f32_lds_kernel"},
    {static_cast<int>(kern::GemmF32Variant::kDataParallelBK32), "f32_dp_64x64x32", 64, 64, 32, 8, 2,
     "gemm_f32_lds_kernel"},
};

constexpr VariantInfo kHalfVariants[] = {
    {static_cast<int>(kern::GemmHalfVariant::kW4), "half_w4_256x256", 256, 256, 32, 4, 1, "gemm_half_tn_w4_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kW4D), "half_w4d_256x256", 256, 256, 64, 4, 1,
     "gemm_half_tn_w4d_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kW4R), "half_w4r_256x256", 256, 256, 64, 4, 1,
     "gemm_half_tn_w4r_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kW4H), "half_w4h_256x256", 256, 256, 64, 4, 1,
     "gemm_half_tn_w4h_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kLds), "half_lds_256x256", 256, 256, 64, 8, 1,
     "gemm_half_tn_lds_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kBig8), "half_big8_256x256", 256, 256, 64, 8, 1, "gemm_half_tn_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kBig4), "half_big4_256x256", 256, 256, 64, 4, 1, "gemm_half_tn_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kMid), "half_mid_128x128", 128, 128, 64, 4, 1, "gemm_half_tn_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kSmall), "half_small_64x64", 64, 64, 64, 4, 1, "gemm_half_tn_kernel"},
    {static_cast<int>(kern::GemmHalfVariant::kSkinny), "half_skinny_16x64", 16, 64, 256, 8, 2, "gemm_skinny_kernel"},
};

struct VariantTable {
  const VariantInfo* first;
  const VariantInfo* last;
  const VariantInfo* begin() const { return first; }
  const VariantInfo* end() const { return last; }
};

VariantTable variants(bool half) {
  return half ? VariantTable{std::begin(kHalfVariants), std::end(kHalfVariants)}
              : VariantTable{std::begin(kF32Variants), std::end(kF32Variants)};
}

TuneEntry entryFor(bool half, int variant) {
  TuneEntry e;
  for (const VariantInfo& v : variants(half)) {
    if (v.variant == variant) {
      e.kernel = v.name;
      e.tile_m = v.tile_m;
      e.tile_n = v.tile_n;
      e.tile_k = v.tile_k;
      e.waves = v.waves;
      e.split_k = v.split_k;
    }
  }
  return e;
}

// A cached entry names a variant this shape can run (else it is ignored).
bool variantFromEntry(const TuneEntry& e, bool half, std::size_t m, int* variant) {
  for (const VariantInfo& v : variants(half)) {
    if (e.kernel == v.name) {
      const bool skinny = v.variant == static_cast<int>(kern::GemmHalfVariant::kSkinny);
      if (half && skinny != (m <= 16)) {
        return false;
      }
      *variant = v.variant;
      return true;
    }
  }
  return false;
}

hipError_t launchGemm(HipContext* ctx, MatMulResident& r, int variant) {
  const int M = static_cast<int>(r.m);
  const int K = static_cast<int>(r.k);
  const int N = static_cast<int>(r.n);
  if (!isHalf(r.dtype)) {
    const int kp = static_cast<int>(roundUp(r.k, kern::kF32GemmBK));
    const int np = static_cast<int>(roundUp(r.n, kern::kF32GemmBN));
    // stream-K: one workgroup per CU (a whole-tile grid may hold two per CU)
    const int groups = ctx->props.multiProcessorCount > 0 ? ctx->props.multiProcessorCount : 256;
    const bool fresh_fail = ctx->gemm_fail.get() == nullptr;
    if (ctx->gemm_part.ensure(static_cast<std::size_t>(groups) * 4096 * sizeof(float)) != Status::kSuccess ||
        ctx->gemm_flags.ensure(static_cast<std::size_t>(groups) * sizeof(int), true) != Status::kSuccess ||
        ctx->gemm_fail.ensure(sizeof(int)) != Status::kSuccess) {
      return hipErrorOutOfMemory;
    }
    if (fresh_fail) {
      *static_cast<int*>(ctx->gemm_fail.get()) = 0;
    }
    kern::StreamKSync sync{ctx->gemm_part.as<float>(), ctx->gemm_flags.as<int>(),
                           static_cast<int*>(ctx->gemm_fail.device()), 0, streamKSpinLimit()};
    if (nextStreamKEpoch(ctx, &sync.epoch) != Status::kSuccess) {
      return hipErrorUnknown;
    }
    return kern::gemmF32Padded(r.a.as<float>(), r.b.as<float>(), r.c.as<float>(), M, N, kp, kp, np, N, sync, groups,
                               static_cast<kern::GemmF32Variant>(variant), ctx->stream);
  }
  const int kp = static_cast<int>(roundUp(r.k, kern::kHalfGemmBK));
  kern::SkinnyWork skinny{nullptr, nullptr, 0, 0, 0};
  if (M <= 16) {
    const int tiles = static_cast<int>(roundUp(r.n, 64) / 64);
    if (ctx->skinny_part.ensure(static_cast<std::size_t>(kern::kSkinnyMaxSplits) * tiles * kern::kSkinnyPartFloats *
                                sizeof(float)) != Status::kSuccess ||
        ctx->skinny_counters.ensure(static_cast<std::size_t>(tiles) * sizeof(int), true) != Status::kSuccess) {
      return hipErrorOutOfMemory;
    }
    skinny = kern::SkinnyWork{ctx->skinny_part.as<float>(), ctx->skinny_counters.as<int>(),
                              static_cast<int>(ctx->skinny_counters.size() / sizeof(int)), kern::kSkinnyMaxSplits,
                              ctx->props.multiProcessorCount > 0 ? ctx->props.multiProcessorCount : 256};
  }
  return kern::gemmHalfTN(r.a.as<uint16_t>(), r.b.as<uint16_t>(), r.c.as<float>(), M, N, kp, kp, kp, N,
                          halfOf(r.dtype), static_cast<kern::GemmHalfVariant>(variant), ctx->stream, &skinny);
}

// Times the candidates round-robin (so clock and thermal drift spread over
// all of them): one warm-up round, then 5 rounds of 2 back-to-back launches
// per candidate timed with HIP events on the context stream; the median per
// candidate counts (the reference's autoTuneTile takes a 5-sample median,
// src/ops/matmul_metal.mm:1687-1710).
Status timeVariants(HipContext* ctx, MatMulResident& r, const std::vector<int>& cands, std::vector<float>* ms) {
  constexpr int kRounds = 5;
  constexpr int kLaunches = 2;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  LC_HIP_TRY(hipEventCreate(&e0));
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return failHip(hipErrorOutOfMemory, "matmul autotune events");
  }
  std::vector<std::vector<float>> samples(cands.size());
  hipError_t e = hipSuccess;
  for (int round = -1; round < kRounds && e == hipSuccess; ++round) {
    for (std::size_t c = 0; c < cands.size() && e == hipSuccess; ++c) {
      e = hipEventRecord(e0, ctx->stream);
      for (int l = 0; l < kLaunches && e == hipSuccess; ++l) {
        e = launchGemm(ctx, r, cands[c]);
      }
      if (e == hipSuccess) e = hipEventRecord(e1, ctx->stream);
      if (e == hipSuccess) e = hipEventSynchronize(e1);
      float t = 0.0f;
      if (e == hipSuccess) e = hipEventElapsedTime(&t, e0, e1);
      if (round >= 0) {
        samples[c].push_back(t);
      }
    }
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (e != hipSuccess) {
    return failHip(e, "matmul autotune");
  }
  ms->clear();
  for (auto& v : samples) {
    std::sort(v.begin(), v.end());
    ms->push_back(v[v.size() / 2]);
  }
  return Status::kSuccess;
}

// Settles r.variant for the shape: a tune-cache entry, else (CJ_MATMUL_AUTOTUNE
// not off) the fastest candidate, else the heuristic; the choice is recorded.
// CJ_HIP_GEMM_F32 / CJ_HIP_GEMM_TILE (sweep overrides) bypass all of it.
Status settleVariant(HipContext* ctx, MatMulResident& r) {
  const bool half = isHalf(r.dtype);
  r.variant = 0;
  if (std::getenv(half ? "CJ_HIP_GEMM_TILE" : "CJ_HIP_GEMM_F32") != nullptr) {
    return Status::kSuccess;
  }
  const std::string arch = baseArch(ctx);
  const int dtype = static_cast<int>(r.dtype);
  TuneEntry known;
  if (tuneLookup(r.m, r.k, r.n, dtype, arch, &known) && variantFromEntry(known, half, r.m, &r.variant)) {
    return Status::kSuccess;
  }
  const int M = static_cast<int>(r.m);
  const int N = static_cast<int>(r.n);
  const int groups = ctx->props.multiProcessorCount > 0 ? ctx->props.multiProcessorCount : 256;
  int best = half ? static_cast<int>(kern::gemmHalfChoose(M, N)) : static_cast<int>(kern::gemmF32Choose(M, N, groups));
  std::vector<int> cands;
  if (!half) {
    cands = {static_cast<int>(kern::GemmF32Variant::kDataParallel), static_cast<int>(kern::GemmF32Variant::kStreamK)};
  } else if (r.m > 16) {
    for (const VariantInfo& v : kHalfVariants) {
      if (v.variant != static_cast<int>(kern::GemmHalfVariant::kSkinny)) {
        cands.push_back(v.variant);
      }
    }
  }
  if (cands.size() > 1 && autotuneEnabled("CJ_MATMUL_AUTOTUNE")) {
    std::vector<float> ms;
    LC_TRY(timeVariants(ctx, r, cands, &ms));
    // The heuristic's choice stays unless another variant is clearly faster
    // (3%: below that the measurement cannot tell them apart).
    float ref_ms = 0.0f;
    for (std::size_t c = 0; c < cands.size(); ++c) {
      if (cands[c] == best) {
        ref_ms = ms[c];
      }
    }
    float best_ms = ref_ms > 0.0f ? ref_ms * 0.97f : 0.0f;
    for (std::size_t c = 0; c < cands.size(); ++c) {
      if (best_ms <= 0.0f || ms[c] < best_ms) {
        best_ms = ms[c];
        best = cands[c];
      }
    }
  }
  r.variant = best;
  tuneRecord(r.m, r.k, r.n, dtype, arch, entryFor(half, best));
  return Status::kSuccess;
}

// Small fp32 calls that upload both operands and download the product (the
// plain matmul2d call) spend most of their time in per-copy overhead: two
// pageable uploads and a pageable download at ~10 us each, and the stream
// sync.  Here A and B are packed into pinned staging and the padding kernels
// read them through its device alias (each value crosses the bus once); after
// the GEMM one kernel copies C into the staging and raises the host-mapped
// completion flag, which the call waits for instead of a stream sync.
constexpr std::size_t kQuickMatMulElems = std::size_t{1} << 18;  // per operand and the product

bool quickMatMulEnabled() {
  static const bool on = [] {
    const char* v = std::getenv("CJ_HIP_MATMUL_QUICK");
    return v == nullptr || std::string(v) != "0";
  }();
  return on;
}

Status matmulQuick(HipContext* ctx, MatMulResident& r, const float* a, const float* b, float* out) {
  const std::size_t na = r.m * r.k, nb = r.k * r.n, nc = r.m * r.n;
  const std::size_t b_at = roundUp(na, 64);  // 256-byte aligned parts
  const std::size_t c_at = roundUp(b_at + nb, 64);
  const std::size_t mp = roundUp(r.m, kern::kF32GemmBM);
  const std::size_t kp = roundUp(r.k, kern::kF32GemmBK);
  const std::size_t np = roundUp(r.n, kern::kF32GemmBN);
  LC_TRY(ctx->pinned.ensure((c_at + nc) * sizeof(float)));
  LC_TRY(r.a.ensure(mp * kp * sizeof(float)));
  LC_TRY(r.b.ensure(kp * np * sizeof(float)));
  LC_TRY(r.c.ensure(nc * sizeof(float)));
  float* stage = static_cast<float*>(ctx->pinned.get());
  float* dev = static_cast<float*>(ctx->pinned.device());
  std::memcpy(stage, a, na * sizeof(float));
  std::memcpy(stage + b_at, b, nb * sizeof(float));
  hipError_t e = kern::padCopyF32(dev, r.a.as<float>(), static_cast<int>(r.m), static_cast<int>(r.k), r.k,
                                  static_cast<int>(mp), static_cast<int>(kp), ctx->stream);
  if (e == hipSuccess) {
    e = kern::padCopyF32(dev + b_at, r.b.as<float>(), static_cast<int>(r.k), static_cast<int>(r.n), r.n,
                         static_cast<int>(kp), static_cast<int>(np), ctx->stream);
  }
  if (e != hipSuccess) {
    return failHip(e, "matmul upload padding");
  }
  r.has_a = r.has_b = true;
  if (!r.tuned) {
    LC_TRY(settleVariant(ctx, r));
    r.tuned = true;
  }
  unsigned* flag_dev = nullptr;
  unsigned* count_dev = nullptr;
  unsigned seq = 0;
  LC_TRY(prepareDoneFlag(ctx, &flag_dev, &count_dev, &seq));
  traceOpDispatch(TraceOp::kMatMul, Device::kHIP, Device::kHIP, false, r.m * r.k * r.n);
  e = launchGemm(ctx, r, r.variant);
  if (e != hipSuccess) {
    return failHip(e, "matmul kernel launch");
  }
  r.has_c = true;
  e = kern::copyOutFlagF32(r.c.as<float>(), dev + c_at, nc, count_dev, flag_dev, seq, ctx->stream);
  if (e != hipSuccess) {
    return failHip(e, "matmul output copy");
  }
  LC_TRY(waitDoneFlag(ctx, seq));
  std::memcpy(out, stage + c_at, nc * sizeof(float));
  return Status::kSuccess;
}

}  // namespace

Status matmulResident(HipContext* ctx, MatMulResident& r, std::size_t m, std::size_t k, std::size_t n,
                      lcDataType dtype, const float* a, const float* b, float* out, const lcMatMulIoPolicy& policy,
                      std::size_t repeat) {
  if ((policy.upload_a && a == nullptr) || (policy.upload_b && b == nullptr) ||
      (policy.download_out && out == nullptr) || m == 0 || k == 0 || n == 0) {
    return fail(Status::kInvalidValue, "matmul: null pointer required by the io policy or zero dimension");
  }
  if (!validDtype(dtype)) {
    return fail(Status::kInvalidValue, "matmul: unknown compute dtype");
  }
  if (m > (1u << 30) / 1 || k > (1u << 30) || n > (1u << 30) || m * k > (std::size_t(1) << 34) ||
      k * n > (std::size_t(1) << 34) || m * n > (std::size_t(1) << 34)) {
    return fail(Status::kNotSupported, "matmul: shape too large");
  }
  if (r.m != m || r.k != k || r.n != n || r.dtype != dtype) {
    r.has_a = r.has_b = r.has_c = false;
    r.tuned = false;
    r.m = m;
    r.k = k;
    r.n = n;
    r.dtype = dtype;
  }
  if ((!policy.upload_a && !r.has_a) || (!policy.upload_b && !r.has_b)) {
    return fail(Status::kInvalidValue, "matmul: no resident input for an operand the policy does not upload");
  }
  if (!isHalf(dtype) && repeat == 1 && policy.upload_a && policy.upload_b && policy.download_out &&
      std::max({m * k, k * n, m * n}) <= kQuickMatMulElems && quickMatMulEnabled()) {
    return matmulQuick(ctx, r, a, b, out);
  }
  if (policy.upload_a) {
    LC_TRY(uploadA(ctx, r, a));
    r.has_a = true;
  }
  if (policy.upload_b) {
    LC_TRY(uploadB(ctx, r, b));
    r.has_b = true;
  }
  LC_TRY(r.c.ensure(m * n * sizeof(float)));
  const std::size_t hint = m * k * n;
  if (!r.tuned && repeat > 0) {
    LC_TRY(settleVariant(ctx, r));
    r.tuned = true;
  }
  for (std::size_t i = 0; i < repeat; ++i) {
    traceOpDispatch(TraceOp::kMatMul, Device::kHIP, Device::kHIP, false, hint);
    const hipError_t e = launchGemm(ctx, r, r.variant);
    if (e != hipSuccess) {
      return failHip(e, "matmul kernel launch");
    }
  }
  r.has_c = true;
  if (policy.download_out && m * n <= kStagedDownloadMax && quickMatMulEnabled()) {
    const StagedOut o{r.c.as<float>(), out, m * n};
    return stagedDownload(ctx, &o, 1);
  }
  if (policy.download_out) {
    LC_TRY(download(ctx, out, r.c.get(), m * n * sizeof(float)));
  }
  if (policy.download_out || policy.synchronize) {
    LC_TRY(syncStream(ctx));
  } else if (repeat > 0) {
    LC_TRY(noteEnqueued(ctx, TraceOp::kMatMul, repeat));
  }
  return Status::kSuccess;
}

namespace {

MatMulResident& globalMatMulResident() {
  static MatMulResident* r = new MatMulResident();  // process lifetime
  return *r;
}

Status matmulPolicyEntry(const float* a, const float* b, float* out, std::size_t m, std::size_t k, std::size_t n,
                         lcDeviceKind device, const lcMatMulIoPolicy& policy, std::size_t repeat,
                         lcDataType dtype) {
  if ((policy.upload_a && a == nullptr) || (policy.upload_b && b == nullptr) ||
      (policy.download_out && out == nullptr) || m == 0 || k == 0 || n == 0) {
    return fail(Status::kInvalidValue, "matmul: null pointer required by the io policy or zero dimension");
  }
  HipContext* ctx = nullptr;
  LC_TRY(requireHip(device, "matmul", &ctx));
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  return matmulResident(ctx, globalMatMulResident(), m, k, n, dtype, a, b, out, policy, repeat);
}

}  // namespace
}  // namespace lchip

using namespace lchip;

struct lcMatMulResidentSession {
  MatMulResident res;
  std::size_t m = 0, k = 0, n = 0;
  lcDataType dtype = LC_DTYPE_F32;
};

namespace {

lcMatMulIoPolicy makePolicy(int ua, int ub, int dl, int sync) {
  lcMatMulIoPolicy p{};
  p.upload_a = ua;
  p.upload_b = ub;
  p.download_out = dl;
  p.synchronize = sync;
  return p;
}

lcError_t sessionCall(lcMatMulResidentSession* s, const float* a, const float* b, float* out,
                      const lcMatMulIoPolicy& p, std::size_t repeat) {
  if (s == nullptr) {
    return toLc(fail(Status::kInvalidValue, "matmul session: null session"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(LC_DEVICE_HIP, "matmul session", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  return toLc(matmulResident(ctx, s->res, s->m, s->k, s->n, s->dtype, a, b, out, p, repeat));
}

}  // namespace

extern "C" {

lcMatMulIoPolicy lcMatMulIoPolicyDefault(void) { return makePolicy(1, 1, 1, 1); }

lcError_t lcMatMul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n, lcDeviceKind device) {
  return toLc(matmulPolicyEntry(a, b, out, m, k, n, device, makePolicy(1, 1, 1, 1), 1, LC_DTYPE_F32));
}

lcError_t lcMatMulWithPolicy(const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                             lcDeviceKind device, const lcMatMulIoPolicy* policy) {
  const lcMatMulIoPolicy p = policy ? *policy : makePolicy(1, 1, 1, 1);
  return toLc(matmulPolicyEntry(a, b, out, m, k, n, device, p, 1, LC_DTYPE_F32));
}

lcError_t lcMatMulWithPolicyBatched(const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                                    lcDeviceKind device, const lcMatMulIoPolicy* policy, size_t repeat_count) {
  if (repeat_count == 0) {
    return toLc(fail(Status::kInvalidValue, "matmul: repeat_count must be > 0"));
  }
  const lcMatMulIoPolicy p = policy ? *policy : makePolicy(1, 1, 1, 1);
  return toLc(matmulPolicyEntry(a, b, out, m, k, n, device, p, repeat_count, LC_DTYPE_F32));
}

lcError_t lcMatMulResidentSessionCreate(size_t m, size_t k, size_t n, lcDataType compute_dtype,
                                        lcMatMulResidentSession** out) {
  if (out == nullptr || m == 0 || k == 0 || n == 0 || !validDtype(compute_dtype)) {
    return toLc(fail(Status::kInvalidValue, "matmul session: invalid arguments"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(LC_DEVICE_HIP, "matmul session", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  auto* s = new lcMatMulResidentSession();
  s->m = m;
  s->k = k;
  s->n = n;
  s->dtype = compute_dtype;
  *out = s;
  return LC_SUCCESS;
}

lcError_t lcMatMulResidentSessionDestroy(lcMatMulResidentSession* s) {
  if (s == nullptr) {
    return LC_INVALID_VALUE;
  }
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx != nullptr) {
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipStreamSynchronize(ctx->stream);
  }
  delete s;
  return LC_SUCCESS;
}

// ops.hpp:207-216 / policy.hpp:37-44: upload both, no download, no sync.
lcError_t lcMatMulResidentSessionStart(lcMatMulResidentSession* s, const float* a, const float* b, float* out) {
  return sessionCall(s, a, b, out, makePolicy(1, 1, 0, 0), 1);
}
// ops.hpp:218-227 / policy.hpp:46-53: launch only.
lcError_t lcMatMulResidentSessionRun(lcMatMulResidentSession* s, const float* a, const float* b, float* out) {
  return sessionCall(s, a, b, out, makePolicy(0, 0, 0, 0), 1);
}
// ops.hpp:229-238 / policy.hpp:55-62: launch, download, sync.
lcError_t lcMatMulResidentSessionFinish(lcMatMulResidentSession* s, const float* a, const float* b, float* out) {
  return sessionCall(s, a, b, out, makePolicy(0, 0, 1, 1), 1);
}
// ops.hpp:240-249 / policy.hpp:64-71: launch, sync, no download.
lcError_t lcMatMulResidentSessionSync(lcMatMulResidentSession* s, const float* a, const float* b, float* out) {
  return sessionCall(s, a, b, out, makePolicy(0, 0, 0, 1), 1);
}
// ops.hpp:251-299: repeat launches over the resident inputs, then sync.  As
// in the reference (upload=false, download=false, sync=true passed to the
// batched backend), the pointers must be non-null but are not read or written;
// finish() downloads the result.
lcError_t lcMatMulResidentSessionRunBatchSync(lcMatMulResidentSession* s, const float* a, const float* b, float* out,
                                              size_t repeat_count) {
  if (repeat_count == 0 || a == nullptr || b == nullptr || out == nullptr) {
    return toLc(fail(Status::kInvalidValue, "matmul session: run_batch_sync needs pointers and repeat_count > 0"));
  }
  return sessionCall(s, nullptr, nullptr, nullptr, makePolicy(0, 0, 0, 1), repeat_count);
}
// ops.hpp:301-352: repeat launches, sync, no download.
lcError_t lcMatMulResidentSessionRunBatchSyncNoDownload(lcMatMulResidentSession* s, const float* a, const float* b,
                                                        float* out, size_t repeat_count) {
  (void)a;
  (void)b;
  (void)out;
  if (repeat_count == 0) {
    return toLc(fail(Status::kInvalidValue, "matmul session: repeat_count must be > 0"));
  }
  return sessionCall(s, nullptr, nullptr, nullptr, makePolicy(0, 0, 0, 1), repeat_count);
}
// ops.hpp:1371-1373: the same with null pointers.
lcError_t lcMatMulResidentSessionRunBatchSyncCachedNoDownload(lcMatMulResidentSession* s, size_t repeat_count) {
  return lcMatMulResidentSessionRunBatchSyncNoDownload(s, nullptr, nullptr, nullptr, repeat_count);
}

lcError_t lcMatMulResidentSessionTimeLaunches(lcMatMulResidentSession* s, size_t count, float* ms_out) {
  if (s == nullptr || count == 0 || ms_out == nullptr) {
    return toLc(fail(Status::kInvalidValue, "matmul session: null session or output, or count 0"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(LC_DEVICE_HIP, "matmul session", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  MatMulResident& r = s->res;
  if (!r.has_a || !r.has_b || r.m != s->m || r.k != s->k || r.n != s->n || r.dtype != s->dtype) {
    return toLc(fail(Status::kInvalidValue, "matmul session: no resident inputs to time (start the session first)"));
  }
  if (!r.tuned) {
    st = settleVariant(ctx, r);
    if (st != Status::kSuccess) {
      return toLc(st);
    }
    r.tuned = true;
  }
  std::vector<hipEvent_t> ev(2 * count, nullptr);
  hipError_t e = hipSuccess;
  for (std::size_t i = 0; i < ev.size() && e == hipSuccess; ++i) {
    e = hipEventCreate(&ev[i]);
  }
  for (std::size_t i = 0; i < count && e == hipSuccess; ++i) {
    e = hipEventRecord(ev[2 * i], ctx->stream);
    if (e == hipSuccess) {
      traceOpDispatch(TraceOp::kMatMul, Device::kHIP, Device::kHIP, false, r.m * r.k * r.n);
      e = launchGemm(ctx, r, r.variant);
    }
    if (e == hipSuccess) {
      e = hipEventRecord(ev[2 * i + 1], ctx->stream);
    }
  }
  if (e == hipSuccess) {
    e = hipStreamSynchronize(ctx->stream);
  }
  for (std::size_t i = 0; i < count && e == hipSuccess; ++i) {
    e = hipEventElapsedTime(&ms_out[i], ev[2 * i], ev[2 * i + 1]);
  }
  for (hipEvent_t x : ev) {
    if (x != nullptr) {
      (void)hipEventDestroy(x);
    }
  }
  if (e != hipSuccess) {
    return toLc(failHip(e, "matmul session: timed launches"));
  }
  r.has_c = true;
  return toLc(syncStream(ctx));
}

lcError_t lcMatMulResidentSessionKernelName(lcMatMulResidentSession* s, char* buf, size_t cap) {
  if (s == nullptr || buf == nullptr || cap == 0) {
    return toLc(fail(Status::kInvalidValue, "matmul session: null session or buffer"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(LC_DEVICE_HIP, "matmul session", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  const bool half = isHalf(s->dtype);
  int v = s->res.tuned ? s->res.variant : 0;
  if (v == 0) {
    const int groups = ctx->props.multiProcessorCount > 0 ? ctx->props.multiProcessorCount : 256;
    v = half ? (s->m <= 16 ? static_cast<int>(kern::GemmHalfVariant::kSkinny)
                           : static_cast<int>(kern::gemmHalfChoose(static_cast<int>(s->m), static_cast<int>(s->n))))
             : static_cast<int>(kern::gemmF32Choose(static_cast<int>(s->m), static_cast<int>(s->n), groups));
  }
  std::string text;
  for (const VariantInfo& info : variants(half)) {
    if (info.variant == v) {
      text = std::string(info.name) + " " + info.hip_kernel;
    }
  }
  if (text.empty()) {
    return toLc(fail(Status::kUnknown, "matmul session: unknown variant"));
  }
  std::snprintf(buf, cap, "%s", text.c_str());
  return LC_SUCCESS;
}

}  // extern "C"
