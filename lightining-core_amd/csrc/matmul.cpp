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
#include <cstring>

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

// The kernel configuration the dispatch below selects for a shape (recorded
// in the tune cache so it can be saved, inspected and reset).
TuneEntry gemmConfig(const MatMulResident& r) {
  TuneEntry e;
  if (!isHalf(r.dtype)) {
    e.kernel = "f32_lds_32x32x2";
    e.tile_m = kern::kF32GemmBM;
    e.tile_n = kern::kF32GemmBN;
    e.tile_k = kern::kF32GemmBK;
    e.waves = 8;
    e.split_k = 2;  // two wave groups per block, one per K half of each stage
  } else if (r.m <= 16) {
    e.kernel = "half_skinny_16x16x32";
    e.tile_m = 16;
    e.tile_n = 32;
    e.tile_k = 32;
    e.waves = 4;
    e.split_k = 4;
  } else {
    // mirrors pick_half_tile() in kernels/gemm.hip
    const auto tiles = [&](std::size_t b) { return ((r.m + b - 1) / b) * ((r.n + b - 1) / b); };
    e.kernel = "half_tn_32x32x16";
    if (tiles(256) >= 256) {
      e.tile_m = e.tile_n = 256;
      e.tile_k = 64;
      e.waves = 8;
    } else if (tiles(128) >= 256) {
      e.tile_m = e.tile_n = 128;
      e.tile_k = 64;
      e.waves = 4;
    } else {
      e.tile_m = e.tile_n = 64;
      e.tile_k = 64;
      e.waves = 4;
    }
  }
  return e;
}

hipError_t launchGemm(HipContext* ctx, MatMulResident& r) {
  const int M = static_cast<int>(r.m);
  const int K = static_cast<int>(r.k);
  const int N = static_cast<int>(r.n);
  if (!isHalf(r.dtype)) {
    const int kp = static_cast<int>(roundUp(r.k, kern::kF32GemmBK));
    const int np = static_cast<int>(roundUp(r.n, kern::kF32GemmBN));
    // stream-K: one workgroup per CU at most (112 KB of LDS each)
    const int groups = ctx->props.multiProcessorCount > 0 ? ctx->props.multiProcessorCount : 256;
    if (ctx->gemm_part.ensure(static_cast<std::size_t>(groups) * 4096 * sizeof(float)) != Status::kSuccess ||
        ctx->gemm_flags.ensure(static_cast<std::size_t>(groups) * sizeof(int), true) != Status::kSuccess) {
      return hipErrorOutOfMemory;
    }
    return kern::gemmF32Padded(r.a.as<float>(), r.b.as<float>(), r.c.as<float>(), M, N, kp, kp, np, N,
                               ctx->gemm_part.as<float>(), ctx->gemm_flags.as<int>(), groups, ctx->stream);
  }
  const int kp = static_cast<int>(roundUp(r.k, kern::kHalfGemmBK));
  return kern::gemmHalfTN(r.a.as<uint16_t>(), r.b.as<uint16_t>(), r.c.as<float>(), M, N, kp, kp, kp, N,
                          halfOf(r.dtype), ctx->stream);
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
    r.m = m;
    r.k = k;
    r.n = n;
    r.dtype = dtype;
  }
  if ((!policy.upload_a && !r.has_a) || (!policy.upload_b && !r.has_b)) {
    return fail(Status::kInvalidValue, "matmul: no resident input for an operand the policy does not upload");
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
  TuneEntry known;
  if (!tuneLookup(m, k, n, static_cast<int>(dtype), ctx->props.gcnArchName, &known)) {
    tuneRecord(m, k, n, static_cast<int>(dtype), ctx->props.gcnArchName, gemmConfig(r));
  }
  for (std::size_t i = 0; i < repeat; ++i) {
    traceOpDispatch(TraceOp::kMatMul, Device::kHIP, Device::kHIP, false, hint);
    const hipError_t e = launchGemm(ctx, r);
    if (e != hipSuccess) {
      return failHip(e, "matmul kernel launch");
    }
  }
  r.has_c = true;
  if (policy.download_out) {
    LC_TRY(download(ctx, out, r.c.get(), m * n * sizeof(float)));
  }
  if (policy.download_out || policy.synchronize) {
    LC_TRY(syncStream(ctx));
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

}  // extern "C"
