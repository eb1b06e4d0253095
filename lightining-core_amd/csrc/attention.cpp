// attention.cpp -- attention front-end for the "hip" device.
//
// Mirrors lightning_core::attentionForwardWithPolicy (reference
// src/attention.cpp:137-201) and AttentionSession (:247-283):
//   * validation: null q/k/v/out or zero dims -> kInvalidValue (:146-148);
//   * workload hint S*S*D (per head) in the op_dispatch trace (:149);
//   * postprocess out = relu?(out*scale + bias), identity skipped (:41-60);
//   * sessions default to synchronize = false, loss_every = 0 (:247-254);
//   * a download always synchronises (the host reads the result).
// The reference's CPU paths (device cpu, the one-shot CPU crossover and the
// kNotSupported -> CPU fallback) belong to the reference's own dispatcher; in
// this library a request that the HIP kernels cannot serve returns an error.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <memory>
#include <vector>

#include "ops_internal.hpp"
#include "tune.hpp"

namespace lchip {

Status requireHip(lcDeviceKind device, const char* op, HipContext** ctx_out) {
  if (!validDevice(device)) {
    return fail(Status::kInvalidValue, std::string(op) + ": unknown device");
  }
  if (device != LC_DEVICE_HIP) {
    return fail(Status::kNotSupported, std::string(op) +
                                           ": this library implements the 'hip' device only; cpu/cuda/metal compute "
                                           "is served by the reference backends");
  }
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx == nullptr) {
    return st;
  }
  *ctx_out = ctx;
  return Status::kSuccess;
}

namespace {

Status uploadAttnTensor(HipContext* ctx, AttnResident& res, const AttnShape& sh, const float* host, DeviceBuffer& dst,
                        bool transpose) {
  const std::size_t n = sh.elems();
  if (!isHalf(sh.dtype)) {
    LC_TRY(dst.ensure(n * sizeof(float)));
    return upload(ctx, dst.get(), host, n * sizeof(float));
  }
  const std::size_t s_pad = sh.sPad();
  LC_TRY(res.stage.ensure(n * sizeof(float)));
  LC_TRY(dst.ensure(sh.bh() * s_pad * sh.head_dim * sizeof(uint16_t)));
  LC_TRY(upload(ctx, res.stage.get(), host, n * sizeof(float)));
  const int S = static_cast<int>(sh.seq_len);
  const int D = static_cast<int>(sh.head_dim);
  const int bh = static_cast<int>(sh.bh());
  hipError_t e;
  if (!transpose) {
    e = kern::convertPad(res.stage.as<float>(), dst.as<uint16_t>(), bh, S, D, D, static_cast<int>(s_pad), D,
                         sh.seq_len * sh.head_dim, s_pad * sh.head_dim, halfOf(sh.dtype), ctx->stream);
  } else {
    e = kern::convertTransposePad(res.stage.as<float>(), dst.as<uint16_t>(), bh, S, D, D, static_cast<int>(s_pad), D,
                                  sh.seq_len * sh.head_dim, s_pad * sh.head_dim, halfOf(sh.dtype), ctx->stream);
  }
  if (e != hipSuccess) {
    return failHip(e, "attention upload conversion");
  }
  return Status::kSuccess;
}

bool sameShape(const AttnShape& a, const AttnShape& b) {
  return a.batch == b.batch && a.heads == b.heads && a.seq_len == b.seq_len && a.head_dim == b.head_dim &&
         a.dtype == b.dtype;
}

bool postIsIdentity(const lcAttentionIoPolicy& p) {
  return p.output_scale == 1.0f && p.output_bias == 0.0f && !p.output_relu;
}

// Median time of each candidate launch, timed round-robin (one warm-up
// round, then 3 rounds; HIP events on the context stream) so that clock
// drift spreads over all candidates.  The reference's forward autotune takes
// a 3-sample median per mode (src/attention_metal.mm:1517-1574).
template <typename Launch>
Status timeCandidates(HipContext* ctx, const std::vector<int>& cands, Launch launch, std::vector<float>* ms) {
  constexpr int kRounds = 3;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  LC_HIP_TRY(hipEventCreate(&e0));
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return failHip(hipErrorOutOfMemory, "attention autotune events");
  }
  std::vector<std::vector<float>> samples(cands.size());
  hipError_t e = hipSuccess;
  for (int round = -1; round < kRounds && e == hipSuccess; ++round) {
    for (std::size_t c = 0; c < cands.size() && e == hipSuccess; ++c) {
      e = hipEventRecord(e0, ctx->stream);
      if (e == hipSuccess) e = launch(cands[c]);
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
    return failHip(e, "attention autotune");
  }
  ms->clear();
  for (auto& v : samples) {
    std::sort(v.begin(), v.end());
    ms->push_back(v[v.size() / 2]);
  }
  return Status::kSuccess;
}

// The heuristic's split count stays unless another is faster by 3%.
int pickSplits(const std::vector<int>& cands, const std::vector<float>& ms, int heuristic) {
  float ref = 0.0f;
  for (std::size_t c = 0; c < cands.size(); ++c) {
    if (cands[c] == heuristic) {
      ref = ms[c];
    }
  }
  int best = heuristic;
  float best_ms = ref > 0.0f ? ref * 0.97f : 0.0f;
  for (std::size_t c = 0; c < cands.size(); ++c) {
    if (best_ms <= 0.0f || ms[c] < best_ms) {
      best_ms = ms[c];
      best = cands[c];
    }
  }
  return best;
}

// The fp32 forward's key splits: on unless CJ_HIP_ATTN_KEY_SPLIT=0 (read
// once; without a workspace every call runs unsplit).
bool keySplitEnabled() {
  static const bool on = [] {
    const char* v = std::getenv("CJ_HIP_ATTN_KEY_SPLIT");
    return v == nullptr || std::string(v) != "0";
  }();
  return on;
}

// The fp32 forward's key-split workspace, grown to at least `floats`.
Status ensureSplitWs(AttnResident& res, std::size_t floats) {
  return floats > 0 && keySplitEnabled() ? res.split_ws.ensure(floats * sizeof(float)) : Status::kSuccess;
}

// Split counts worth timing for one head: the valid ones (LDS limits) up to
// the number of 32-key tiles.
std::vector<int> splitCandidates(int S, int D) {
  const int tiles = (S + 31) / 32;
  std::vector<int> c;
  for (int ks = 1; ks <= 8; ks *= 2) {
    if (kern::attentionF32Splits(1, S, D, ks) == ks && (ks == 1 || ks <= tiles)) {
      c.push_back(ks);
    }
  }
  // The 16-query forward / 16-key dV kernels (D <= 64, D % 4 == 0; session
  // buffers are 16-byte aligned) for one head of a thousand keys or fewer.
  if (S <= 1024 && kern::attentionF32Splits(1, S, D, kern::kAttnF32Q16) == kern::kAttnF32Q16) {
    c.push_back(kern::kAttnF32Q16);
  }
  return c;
}

// The fp32 single-head forward's split count for this key: the tune cache,
// else the fastest candidate (CJ_ATTN_AUTOTUNE not off), else the heuristic
// (src/attention_metal.mm:1483-1583 is the reference's forward autotune).
Status forwardSplits(HipContext* ctx, AttnResident& res, const AttnShape& sh, const lcAttentionIoPolicy& policy,
                     int* splits) {
  AttnTuneKey key;
  key.kind = 'F';
  key.arch = baseArch(ctx);
  key.seq = sh.seq_len;
  key.dim = sh.head_dim;
  key.causal = sh.causal ? 1 : 0;
  key.resident_hint = (!policy.upload_q && !policy.upload_k && !policy.upload_v && !policy.download_out) ? 1 : 0;
  key.sync_hint = policy.synchronize ? 1 : 0;
  if (attnTuneLookup(key, splits)) {
    return Status::kSuccess;
  }
  const int S = static_cast<int>(sh.seq_len);
  const int D = static_cast<int>(sh.head_dim);
  int best = kern::attentionF32DefaultSplits(1, S, D);
  const std::vector<int> cands = splitCandidates(S, D);
  if (cands.size() > 1 && autotuneEnabled("CJ_ATTN_AUTOTUNE")) {
    std::size_t ws = 0;
    for (int ks : cands) {
      ws = std::max(ws, kern::attentionF32WorkspaceFloats(1, S, D, ks));
    }
    LC_TRY(ensureSplitWs(res, ws));
    std::vector<float> ms;
    LC_TRY(timeCandidates(
        ctx, cands,
        [&](int ks) {
          return kern::attentionF32(res.q.as<float>(), res.k.as<float>(), res.v.as<float>(), res.out.as<float>(), 1,
                                    S, D, sh.causal, policy.output_scale, policy.output_bias, policy.output_relu,
                                    nullptr, ctx->stream, ks, nullptr, nullptr, 0, res.split_ws.as<float>(),
                                    res.split_ws.size() / sizeof(float));
        },
        &ms));
    best = pickSplits(cands, ms, best);
  }
  attnTuneRecord(key, best);
  *splits = best;
  return Status::kSuccess;
}

// The train step's dV split count (T rows; src/attention_metal.mm:1700-1830
// tunes the reference's train modes).  Candidates run on a copy of V: the
// kernel updates V in place.
Status trainSplits(HipContext* ctx, AttnResident& res, const AttnShape& sh, const lcAttentionIoPolicy& policy,
                   bool compute_loss, float lr, int* splits) {
  AttnTuneKey key;
  key.kind = 'T';
  key.arch = baseArch(ctx);
  key.seq = sh.seq_len;
  key.dim = sh.head_dim;
  key.causal = sh.causal ? 1 : 0;
  key.resident_hint = (!policy.upload_q && !policy.upload_k && !policy.upload_v && !policy.download_v) ? 1 : 0;
  key.sync_hint = policy.synchronize ? 1 : 0;
  key.compute_loss = compute_loss ? 1 : 0;
  if (attnTuneLookup(key, splits)) {
    return Status::kSuccess;
  }
  const int S = static_cast<int>(sh.seq_len);
  const int D = static_cast<int>(sh.head_dim);
  int best = kern::attentionF32DefaultSplits(1, S, D);
  const std::vector<int> cands = splitCandidates(S, D);
  if (cands.size() > 1 && autotuneEnabled("CJ_ATTN_AUTOTUNE")) {
    const std::size_t bytes = sh.elems() * sizeof(float);
    LC_TRY(res.v_scratch.ensure(bytes));
    LC_HIP_TRY(hipMemcpyAsync(res.v_scratch.get(), res.v.get(), bytes, hipMemcpyDeviceToDevice, ctx->stream));
    std::size_t ws = 0;
    for (int ks : cands) {
      ws = std::max(ws, kern::attentionDvWorkspaceFloats(1, S, D, ks));
    }
    LC_TRY(ensureSplitWs(res, ws));
    std::vector<float> ms;
    LC_TRY(timeCandidates(
        ctx, cands,
        [&](int ks) {
          return kern::attentionDvUpdateF32(res.q.as<float>(), res.k.as<float>(), res.v_scratch.as<float>(),
                                            res.out.as<float>(), res.target.as<float>(), res.stats.as<float>(), 1, S,
                                            D, sh.causal, lr, ctx->stream, ks, res.split_ws.as<float>(),
                                            res.split_ws.size() / sizeof(float));
        },
        &ms));
    best = pickSplits(cands, ms, best);
  }
  attnTuneRecord(key, best);
  *splits = best;
  return Status::kSuccess;
}

// Small one-head fp32 calls that upload every input and download the output
// (the plain attention2d call) spend most of their time in per-copy
// overhead: three pageable uploads, a pageable download and a stream sync,
// ~10 us each at 64 KB.  Here the inputs are packed into pinned staging and
// one copy kernel reads them through its device alias into the resident
// buffers (a DMA copy from pinned memory still costs ~10 us per copy at these
// sizes); the attention kernel writes the output straight into the staging
// and raises the host-mapped completion flag, which the call waits for
// instead of a stream sync.
constexpr std::size_t kQuickAttnElems = std::size_t{1} << 16;  // S * D per tensor

bool quickAttnEnabled() {
  static const bool on = [] {
    const char* v = std::getenv("CJ_HIP_ATTN_QUICK");
    return v == nullptr || std::string(v) != "0";
  }();
  return on;
}

Status attentionForwardQuick(HipContext* ctx, AttnResident& res, const AttnShape& sh, const float* q,
                             const float* k, const float* v, float* out, const lcAttentionIoPolicy& policy) {
  const std::size_t n = sh.elems();
  const std::size_t bytes = n * sizeof(float);
  const std::size_t out_at = roundUp(3 * n, 64);  // 256-byte aligned output
  LC_TRY(ctx->pinned.ensure((out_at + n) * sizeof(float)));
  LC_TRY(res.q.ensure(bytes));
  LC_TRY(res.k.ensure(bytes));
  LC_TRY(res.v.ensure(bytes));
  LC_TRY(res.out.ensure(bytes));
  float* stage = static_cast<float*>(ctx->pinned.get());
  std::memcpy(stage, q, bytes);
  std::memcpy(stage + n, k, bytes);
  std::memcpy(stage + 2 * n, v, bytes);
  const float* dev = static_cast<const float*>(ctx->pinned.device());
  kern::CopySegsF32 in{};
  in.seg[0] = kern::CopySegF32{dev, res.q.as<float>(), n};
  in.seg[1] = kern::CopySegF32{dev + n, res.k.as<float>(), n};
  in.seg[2] = kern::CopySegF32{dev + 2 * n, res.v.as<float>(), n};
  in.count = 3;
  const hipError_t ce = kern::copySegsF32(in, ctx->stream);
  if (ce != hipSuccess) {
    return failHip(ce, "attention input copy");
  }
  res.has_q = res.has_k = res.has_v = true;
  int splits = 0;
  LC_TRY(forwardSplits(ctx, res, sh, policy, &splits));
  unsigned* flag_dev = nullptr;
  unsigned* count_dev = nullptr;
  unsigned seq = 0;
  const int S = static_cast<int>(sh.seq_len);
  const int D = static_cast<int>(sh.head_dim);
  LC_TRY(ensureSplitWs(res, kern::attentionF32WorkspaceFloats(1, S, D, splits)));
  LC_TRY(prepareDoneFlag(ctx, &flag_dev, &count_dev, &seq));
  traceOpDispatch(TraceOp::kAttentionForward, Device::kHIP, Device::kHIP, false, sh.seq_len * sh.seq_len * sh.head_dim);
  const hipError_t e = kern::attentionF32(res.q.as<float>(), res.k.as<float>(), res.v.as<float>(),
                                          static_cast<float*>(ctx->pinned.device()) + out_at, 1, S, D, sh.causal,
                                          policy.output_scale, policy.output_bias, policy.output_relu, nullptr,
                                          ctx->stream, splits, count_dev, flag_dev, seq, res.split_ws.as<float>(),
                                          res.split_ws.size() / sizeof(float));
  if (e != hipSuccess) {
    return failHip(e, "attention kernel launch");
  }
  LC_TRY(waitDoneFlag(ctx, seq));
  std::memcpy(out, stage + out_at, bytes);
  res.has_out = false;  // the output went to the staging, not to res.out
  return Status::kSuccess;
}

}  // namespace

Status attentionForwardResident(HipContext* ctx, AttnResident& res, const AttnShape& sh, const float* q,
                                const float* k, const float* v, float* out, const lcAttentionIoPolicy& policy,
                                std::size_t repeat) {
  if (sh.seq_len == 0 || sh.head_dim == 0 || sh.bh() == 0) {
    return fail(Status::kInvalidValue, "attention: zero dimension");
  }
  if ((policy.upload_q && q == nullptr) || (policy.upload_k && k == nullptr) || (policy.upload_v && v == nullptr) ||
      (policy.download_out && out == nullptr)) {
    return fail(Status::kInvalidValue, "attention: null pointer required by the io policy");
  }
  if (isHalf(sh.dtype) && sh.head_dim != 64 && sh.head_dim != 128) {
    return fail(Status::kNotSupported, "attention: 16-bit path supports head_dim 64 or 128");
  }
  if (!isHalf(sh.dtype) && sh.head_dim > 256) {
    return fail(Status::kNotSupported, "attention: fp32 path supports head_dim <= 256");
  }
  if (sh.seq_len > (1u << 24) || sh.bh() > 65535u * 64u) {
    return fail(Status::kNotSupported, "attention: shape too large");
  }
  if (!sameShape(res.shape, sh)) {
    res.has_q = res.has_k = res.has_v = res.has_out = false;
    res.shape = sh;
  }
  if ((!policy.upload_q && !res.has_q) || (!policy.upload_k && !res.has_k) || (!policy.upload_v && !res.has_v)) {
    return fail(Status::kInvalidValue, "attention: no resident input for a tensor the policy does not upload");
  }

  const bool half = isHalf(sh.dtype);
  if (!half && sh.bh() == 1 && repeat == 1 && policy.upload_q && policy.upload_k && policy.upload_v &&
      policy.download_out && sh.elems() <= kQuickAttnElems && quickAttnEnabled()) {
    return attentionForwardQuick(ctx, res, sh, q, k, v, out, policy);
  }
  if (policy.upload_q) {
    LC_TRY(uploadAttnTensor(ctx, res, sh, q, res.q, false));
    res.has_q = true;
  }
  if (policy.upload_k) {
    LC_TRY(uploadAttnTensor(ctx, res, sh, k, res.k, false));
    res.has_k = true;
  }
  if (policy.upload_v) {
    LC_TRY(uploadAttnTensor(ctx, res, sh, v, res.v, half));
    res.has_v = true;
  }
  const std::size_t n = sh.elems();
  LC_TRY(res.out.ensure(n * sizeof(float)));

  const int S = static_cast<int>(sh.seq_len);
  const int D = static_cast<int>(sh.head_dim);
  const int bh = static_cast<int>(sh.bh());
  const std::size_t hint = sh.seq_len * sh.seq_len * sh.head_dim;
  int splits = 0;  // batched fp32 heads keep the heuristic (the cache keys one head)
  if (!half && bh == 1 && repeat > 0) {
    LC_TRY(forwardSplits(ctx, res, sh, policy, &splits));
  }
  if (!half) {
    LC_TRY(ensureSplitWs(res, kern::attentionF32WorkspaceFloats(bh, S, D, splits)));
  }
  for (std::size_t r = 0; r < repeat; ++r) {
    traceOpDispatch(TraceOp::kAttentionForward, Device::kHIP, Device::kHIP, false, hint);
    hipError_t e;
    if (!half) {
      e = kern::attentionF32(res.q.as<float>(), res.k.as<float>(), res.v.as<float>(), res.out.as<float>(), bh, S, D,
                             sh.causal, policy.output_scale, policy.output_bias, policy.output_relu, nullptr,
                             ctx->stream, splits, nullptr, nullptr, 0, res.split_ws.as<float>(),
                             res.split_ws.size() / sizeof(float));
    } else {
      e = kern::attentionHalf(res.q.as<uint16_t>(), res.k.as<uint16_t>(), res.v.as<uint16_t>(), res.out.as<float>(),
                              nullptr, static_cast<int>(sh.heads), bh, S, static_cast<int>(sh.sPad()), D, sh.causal,
                              halfOf(sh.dtype), ctx->stream);
      if (e == hipSuccess && !postIsIdentity(policy)) {
        e = kern::postprocessF32(res.out.as<float>(), n, policy.output_scale, policy.output_bias, policy.output_relu,
                                 ctx->stream);
      }
    }
    if (e != hipSuccess) {
      return failHip(e, "attention kernel launch");
    }
  }
  res.has_out = true;
  if (policy.download_out && n <= kStagedDownloadMax && quickAttnEnabled()) {
    const StagedOut o{res.out.as<float>(), out, n};
    return stagedDownload(ctx, &o, 1);
  }
  if (policy.download_out) {
    LC_TRY(download(ctx, out, res.out.get(), n * sizeof(float)));
  }
  if (policy.download_out || policy.synchronize) {
    LC_TRY(syncStream(ctx));
  } else if (repeat > 0) {
    LC_TRY(noteEnqueued(ctx, TraceOp::kAttentionForward, repeat));
  }
  return Status::kSuccess;
}

Status attentionTrainResident(HipContext* ctx, AttnResident& res, const AttnShape& sh, const float* q,
                              const float* k, float* v, const float* target, float* out, float learning_rate,
                              float* loss_out, const lcAttentionIoPolicy& policy) {
  // src/attention.cpp:229-232: every pointer, both dims and a positive
  // learning rate are required, whatever the policy.
  if (q == nullptr || k == nullptr || v == nullptr || target == nullptr || out == nullptr || sh.seq_len == 0 ||
      sh.head_dim == 0 || !(learning_rate > 0.0f)) {
    return fail(Status::kInvalidValue, "attention train step: null pointer, zero dimension or learning_rate <= 0");
  }
  if (isHalf(sh.dtype) || sh.bh() != 1) {
    return fail(Status::kNotSupported, "attention train step: fp32, one head (the reference's [S, D] step)");
  }
  if (sh.head_dim > 256 || sh.seq_len > (1u << 24)) {
    return fail(Status::kNotSupported, "attention train step: head_dim <= 256");
  }
  if (!sameShape(res.shape, sh)) {
    res.has_q = res.has_k = res.has_v = res.has_out = res.has_target = false;
    res.shape = sh;
  }
  if ((!policy.upload_q && !res.has_q) || (!policy.upload_k && !res.has_k) || (!policy.upload_v && !res.has_v) ||
      (!policy.upload_target && !res.has_target)) {
    return fail(Status::kInvalidValue, "attention train step: no resident input for a tensor the policy does not upload");
  }
  const std::size_t n = sh.elems();
  const std::size_t bytes = n * sizeof(float);
  // Plain steps of small problems (every input uploaded, out and V downloaded):
  // staged through pinned memory by copy kernels, the wait on the completion
  // flag, as the plain forward (attentionForwardQuick).
  const bool quick = policy.upload_q && policy.upload_k && policy.upload_v && policy.upload_target &&
                     policy.download_out && policy.download_v && n <= kQuickAttnElems && quickAttnEnabled();
  const std::size_t n4 = roundUp(n, 64);  // 256-byte aligned staging slots
  float* stage = nullptr;
  const float* stage_dev = nullptr;
  if (quick) {
    LC_TRY(ctx->pinned.ensure((6 * n4 + 64) * sizeof(float)));
    stage = static_cast<float*>(ctx->pinned.get());
    stage_dev = static_cast<const float*>(ctx->pinned.device());
    std::memcpy(stage, q, bytes);
    std::memcpy(stage + n4, k, bytes);
    std::memcpy(stage + 2 * n4, v, bytes);
    std::memcpy(stage + 3 * n4, target, bytes);
  }
  if (policy.upload_q) {
    LC_TRY(res.q.ensure(bytes));
    if (!quick) LC_TRY(upload(ctx, res.q.get(), q, bytes));
    res.has_q = true;
  }
  if (policy.upload_k) {
    LC_TRY(res.k.ensure(bytes));
    if (!quick) LC_TRY(upload(ctx, res.k.get(), k, bytes));
    res.has_k = true;
  }
  if (policy.upload_v) {
    LC_TRY(res.v.ensure(bytes));
    if (!quick) LC_TRY(upload(ctx, res.v.get(), v, bytes));
    res.has_v = true;
  }
  if (policy.upload_target) {
    LC_TRY(res.target.ensure(bytes));
    if (!quick) LC_TRY(upload(ctx, res.target.get(), target, bytes));
    res.has_target = true;
  }
  if (quick) {
    kern::CopySegsF32 in{};
    in.seg[0] = kern::CopySegF32{stage_dev, res.q.as<float>(), n};
    in.seg[1] = kern::CopySegF32{stage_dev + n4, res.k.as<float>(), n};
    in.seg[2] = kern::CopySegF32{stage_dev + 2 * n4, res.v.as<float>(), n};
    in.seg[3] = kern::CopySegF32{stage_dev + 3 * n4, res.target.as<float>(), n};
    in.count = 4;
    const hipError_t ce = kern::copySegsF32(in, ctx->stream);
    if (ce != hipSuccess) {
      return failHip(ce, "attention train step input copy");
    }
  }
  LC_TRY(res.out.ensure(bytes));
  LC_TRY(res.stats.ensure(sh.seq_len * 2 * sizeof(float)));
  // loss, the reduction's partials, its counter (zero at allocation, left at zero by every launch)
  LC_TRY(res.loss.ensure((2 + kern::kMseLossMaxBlocks) * sizeof(float), true));
  const int S = static_cast<int>(sh.seq_len);
  const int D = static_cast<int>(sh.head_dim);
  // The step's forward has no postprocess (the reference applies it only in
  // attentionForwardWithPolicy, src/attention.cpp:41-60).
  LC_TRY(ensureSplitWs(res, kern::attentionF32WorkspaceFloats(1, S, D, 0)));
  hipError_t e = kern::attentionF32(res.q.as<float>(), res.k.as<float>(), res.v.as<float>(), res.out.as<float>(), 1,
                                    S, D, sh.causal, 1.0f, 0.0f, 0, res.stats.as<float>(), ctx->stream, 0, nullptr,
                                    nullptr, 0, res.split_ws.as<float>(), res.split_ws.size() / sizeof(float));
  if (e == hipSuccess && loss_out != nullptr) {
    e = kern::mseLossF32(res.out.as<float>(), res.target.as<float>(), n,
                         1.0f / static_cast<float>(sh.seq_len * sh.head_dim), res.loss.as<float>(), ctx->stream,
                         res.loss.as<float>() + 1,
                         reinterpret_cast<unsigned*>(res.loss.as<float>() + 1 + kern::kMseLossMaxBlocks));
  }
  if (e != hipSuccess) {
    return failHip(e, "attention train step launch");
  }
  int splits = 0;
  LC_TRY(trainSplits(ctx, res, sh, policy, loss_out != nullptr, learning_rate, &splits));
  LC_TRY(ensureSplitWs(res, kern::attentionDvWorkspaceFloats(1, S, D, splits)));
  e = kern::attentionDvUpdateF32(res.q.as<float>(), res.k.as<float>(), res.v.as<float>(), res.out.as<float>(),
                                 res.target.as<float>(), res.stats.as<float>(), 1, S, D, sh.causal, learning_rate,
                                 ctx->stream, splits, res.split_ws.as<float>(), res.split_ws.size() / sizeof(float));
  if (e != hipSuccess) {
    return failHip(e, "attention train step launch");
  }
  res.has_out = true;
  if (quick) {
    unsigned* flag_dev = nullptr;
    unsigned* count_dev = nullptr;
    unsigned seq = 0;
    LC_TRY(prepareDoneFlag(ctx, &flag_dev, &count_dev, &seq));
    float* odev = static_cast<float*>(ctx->pinned.device());
    kern::CopySegsF32 outs{};
    outs.seg[0] = kern::CopySegF32{res.out.as<float>(), odev + 4 * n4, n};
    outs.seg[1] = kern::CopySegF32{res.v.as<float>(), odev + 5 * n4, n};
    outs.seg[2] = kern::CopySegF32{res.loss.as<float>(), odev + 6 * n4, 1};
    outs.count = loss_out != nullptr ? 3 : 2;
    const hipError_t ce = kern::copySegsF32(outs, ctx->stream, count_dev, flag_dev, seq);
    if (ce != hipSuccess) {
      return failHip(ce, "attention train step output copy");
    }
    LC_TRY(waitDoneFlag(ctx, seq));
    std::memcpy(out, stage + 4 * n4, bytes);
    std::memcpy(v, stage + 5 * n4, bytes);
    if (loss_out != nullptr) {
      *loss_out = stage[6 * n4];
    }
    return Status::kSuccess;
  }
  if ((policy.download_out || policy.download_v || loss_out != nullptr) && quickAttnEnabled() &&
      (n <= kStagedDownloadMax || (!policy.download_out && !policy.download_v))) {
    StagedOut o[3];
    int count = 0;
    if (policy.download_out) o[count++] = StagedOut{res.out.as<float>(), out, n};
    if (policy.download_v) o[count++] = StagedOut{res.v.as<float>(), v, n};
    if (loss_out != nullptr) o[count++] = StagedOut{res.loss.as<float>(), loss_out, 1};
    return stagedDownload(ctx, o, count);
  }
  if (policy.download_out) {
    LC_TRY(download(ctx, out, res.out.get(), bytes));
  }
  if (policy.download_v) {
    LC_TRY(download(ctx, v, res.v.get(), bytes));
  }
  if (loss_out != nullptr) {
    LC_TRY(download(ctx, loss_out, res.loss.get(), sizeof(float)));
  }
  if (policy.download_out || policy.download_v || loss_out != nullptr || policy.synchronize) {
    LC_TRY(syncStream(ctx));
  } else {
    LC_TRY(noteEnqueued(ctx, TraceOp::kAttentionForward, 1));
  }
  return Status::kSuccess;
}

namespace {

AttnResident& globalAttnResident() {
  static AttnResident* r = new AttnResident();  // process lifetime, like the reference's global context
  return *r;
}

Status attentionOneShot(const float* q, const float* k, const float* v, float* out, const AttnShape& sh,
                        lcDeviceKind device, const lcAttentionIoPolicy* policy_in) {
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || sh.seq_len == 0 || sh.head_dim == 0 ||
      sh.bh() == 0) {
    return fail(Status::kInvalidValue, "attention: null pointer or zero dimension");
  }
  if (!validDtype(sh.dtype)) {
    return fail(Status::kInvalidValue, "attention: unknown compute dtype");
  }
  HipContext* ctx = nullptr;
  LC_TRY(requireHip(device, "attention", &ctx));
  const lcAttentionIoPolicy policy = policy_in ? *policy_in : lcAttentionIoPolicyDefault();
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  return attentionForwardResident(ctx, globalAttnResident(), sh, q, k, v, out, policy, 1);
}

// src/attention.cpp:12-39 (autoLossEveryForShape / resolveLossEvery).
int resolveLossEvery(const AttnShape& sh, const lcAttentionIoPolicy& policy) {
  if (policy.loss_every == 0) {
    const std::size_t s = sh.seq_len;
    const std::size_t d = sh.head_dim;
    if (s == 256 && d == 64) {
      return 32;
    }
    if (s == 256 && d == 128) {
      return 16;
    }
    if ((s == 512 || s == 1024) && (d == 64 || d == 128)) {
      return 8;
    }
    return 4;
  }
  return policy.loss_every > 1 ? policy.loss_every : 1;
}

Status attentionTrainOneShot(const float* q, const float* k, float* v, const float* target, float* out, float lr,
                             const lcAttentionConfig* cfg, lcDeviceKind device, float* loss_out,
                             const lcAttentionIoPolicy* policy_in) {
  if (cfg == nullptr) {
    return fail(Status::kInvalidValue, "attention train step: null config");
  }
  AttnShape sh;
  sh.seq_len = cfg->seq_len;
  sh.head_dim = cfg->head_dim;
  sh.causal = cfg->causal != 0;
  if (q == nullptr || k == nullptr || v == nullptr || target == nullptr || out == nullptr || sh.seq_len == 0 ||
      sh.head_dim == 0 || !(lr > 0.0f)) {
    return fail(Status::kInvalidValue, "attention train step: null pointer, zero dimension or learning_rate <= 0");
  }
  HipContext* ctx = nullptr;
  LC_TRY(requireHip(device, "attention train step", &ctx));
  const lcAttentionIoPolicy policy = policy_in ? *policy_in : lcAttentionIoPolicyDefault();
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  return attentionTrainResident(ctx, globalAttnResident(), sh, q, k, v, target, out, lr, loss_out, policy);
}

}  // namespace
}  // namespace lchip

using namespace lchip;

struct lcAttentionSession {
  AttnShape shape;
  lcDeviceKind device = LC_DEVICE_HIP;
  lcAttentionIoPolicy default_policy{};
  AttnResident res;
  // AttentionSession train state (attention.hpp:120-128): sampled-loss
  // bookkeeping of trainStepWithPolicy.
  std::size_t train_step_count = 0;
  float last_loss = 0.0f;
  bool has_last_loss = false;
};

extern "C" {

lcAttentionIoPolicy lcAttentionIoPolicyDefault(void) {
  lcAttentionIoPolicy p{};
  p.upload_q = p.upload_k = p.upload_v = p.upload_target = 1;
  p.download_out = p.download_v = 1;
  p.synchronize = 1;
  p.loss_every = 1;
  p.output_scale = 1.0f;
  p.output_bias = 0.0f;
  p.output_relu = 0;
  return p;
}

const char* lcAttentionImplementationName(lcDeviceKind device) {
  if (device == LC_DEVICE_HIP && hipAvailable()) {
    return "custom-hip-mfma-flash";
  }
  return "unavailable";
}

lcError_t lcAttentionForward(const float* q, const float* k, const float* v, float* out, const lcAttentionConfig* cfg,
                             lcDeviceKind device) {
  return lcAttentionForwardWithPolicy(q, k, v, out, cfg, device, nullptr);
}

lcError_t lcAttentionForwardWithPolicy(const float* q, const float* k, const float* v, float* out,
                                       const lcAttentionConfig* cfg, lcDeviceKind device,
                                       const lcAttentionIoPolicy* policy) {
  if (cfg == nullptr) {
    return toLc(fail(Status::kInvalidValue, "attention: null config"));
  }
  AttnShape sh;
  sh.seq_len = cfg->seq_len;
  sh.head_dim = cfg->head_dim;
  sh.causal = cfg->causal != 0;
  return toLc(attentionOneShot(q, k, v, out, sh, device, policy));
}

lcError_t lcAttentionForwardBatched(const float* q, const float* k, const float* v, float* out,
                                    const lcAttentionBatchedConfig* cfg, lcDeviceKind device,
                                    const lcAttentionIoPolicy* policy) {
  if (cfg == nullptr) {
    return toLc(fail(Status::kInvalidValue, "attention: null config"));
  }
  AttnShape sh;
  sh.batch = cfg->batch;
  sh.heads = cfg->heads;
  sh.seq_len = cfg->seq_len;
  sh.head_dim = cfg->head_dim;
  sh.causal = cfg->causal != 0;
  sh.dtype = cfg->compute_dtype;
  return toLc(attentionOneShot(q, k, v, out, sh, device, policy));
}

static lcError_t createSession(const AttnShape& sh, lcDeviceKind device, lcAttentionSession** out) {
  if (out == nullptr || sh.seq_len == 0 || sh.head_dim == 0 || sh.bh() == 0 || !validDtype(sh.dtype)) {
    return toLc(fail(Status::kInvalidValue, "attention session: invalid arguments"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(device, "attention session", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  auto* s = new lcAttentionSession();
  s->shape = sh;
  s->device = device;
  s->default_policy = lcAttentionIoPolicyDefault();
  // Session defaults target repeated execution (reference src/attention.cpp:249-253).
  s->default_policy.synchronize = 0;
  s->default_policy.loss_every = 0;
  s->res.shape = sh;
  *out = s;
  return LC_SUCCESS;
}

lcError_t lcAttentionSessionCreate(const lcAttentionConfig* cfg, lcDeviceKind device, lcAttentionSession** out) {
  if (cfg == nullptr) {
    return toLc(fail(Status::kInvalidValue, "attention session: null config"));
  }
  AttnShape sh;
  sh.seq_len = cfg->seq_len;
  sh.head_dim = cfg->head_dim;
  sh.causal = cfg->causal != 0;
  return createSession(sh, device, out);
}

lcError_t lcAttentionSessionCreateBatched(const lcAttentionBatchedConfig* cfg, lcDeviceKind device,
                                          lcAttentionSession** out) {
  if (cfg == nullptr) {
    return toLc(fail(Status::kInvalidValue, "attention session: null config"));
  }
  AttnShape sh;
  sh.batch = cfg->batch;
  sh.heads = cfg->heads;
  sh.seq_len = cfg->seq_len;
  sh.head_dim = cfg->head_dim;
  sh.causal = cfg->causal != 0;
  sh.dtype = cfg->compute_dtype;
  return createSession(sh, device, out);
}

lcError_t lcAttentionSessionDestroy(lcAttentionSession* session) {
  if (session == nullptr) {
    return LC_INVALID_VALUE;
  }
  Status st = Status::kSuccess;
  HipContext* ctx = hipContext(&st);
  if (ctx != nullptr) {
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    (void)hipStreamSynchronize(ctx->stream);  // no kernel may still use the buffers
    delete session;
  } else {
    delete session;
  }
  return LC_SUCCESS;
}

lcError_t lcAttentionSessionSetDefaultPolicy(lcAttentionSession* session, const lcAttentionIoPolicy* policy) {
  if (session == nullptr || policy == nullptr) {
    return LC_INVALID_VALUE;
  }
  session->default_policy = *policy;
  return LC_SUCCESS;
}

lcError_t lcAttentionSessionGetDefaultPolicy(const lcAttentionSession* session, lcAttentionIoPolicy* out) {
  if (session == nullptr || out == nullptr) {
    return LC_INVALID_VALUE;
  }
  *out = session->default_policy;
  return LC_SUCCESS;
}

lcError_t lcAttentionSessionForwardWithPolicy(lcAttentionSession* session, const float* q, const float* k,
                                              const float* v, float* out, const lcAttentionIoPolicy* policy) {
  if (session == nullptr || policy == nullptr) {
    return toLc(fail(Status::kInvalidValue, "attention session: null session or policy"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(session->device, "attention session", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  return toLc(attentionForwardResident(ctx, session->res, session->shape, q, k, v, out, *policy, 1));
}

lcError_t lcAttentionSessionForward(lcAttentionSession* session, const float* q, const float* k, const float* v,
                                    float* out) {
  if (session == nullptr) {
    return LC_INVALID_VALUE;
  }
  return lcAttentionSessionForwardWithPolicy(session, q, k, v, out, &session->default_policy);
}

lcError_t lcAttentionSessionRunCached(lcAttentionSession* session, size_t repeat_count) {
  if (session == nullptr || repeat_count == 0) {
    return toLc(fail(Status::kInvalidValue, "attention session: null session or zero repeat"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(session->device, "attention session", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  lcAttentionIoPolicy p = session->default_policy;
  p.upload_q = p.upload_k = p.upload_v = 0;
  p.download_out = 0;
  p.synchronize = 1;
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  return toLc(attentionForwardResident(ctx, session->res, session->shape, nullptr, nullptr, nullptr, nullptr, p,
                                       repeat_count));
}

lcError_t lcAttentionTrainStep(const float* q, const float* k, float* v, const float* target, float* out,
                               float learning_rate, const lcAttentionConfig* cfg, lcDeviceKind device,
                               float* loss_out) {
  return toLc(attentionTrainOneShot(q, k, v, target, out, learning_rate, cfg, device, loss_out, nullptr));
}

lcError_t lcAttentionTrainStepWithPolicy(const float* q, const float* k, float* v, const float* target, float* out,
                                         float learning_rate, const lcAttentionConfig* cfg, lcDeviceKind device,
                                         float* loss_out, const lcAttentionIoPolicy* policy) {
  if (policy == nullptr) {
    return toLc(fail(Status::kInvalidValue, "attention train step: null policy"));
  }
  return toLc(attentionTrainOneShot(q, k, v, target, out, learning_rate, cfg, device, loss_out, policy));
}

lcError_t lcAttentionSessionTrainStepWithPolicy(lcAttentionSession* session, const float* q, const float* k,
                                                float* v, const float* target, float* out, float learning_rate,
                                                float* loss_out, const lcAttentionIoPolicy* policy) {
  if (session == nullptr || policy == nullptr) {
    return toLc(fail(Status::kInvalidValue, "attention session: null session or policy"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(session->device, "attention session train step", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  // src/attention.cpp:298-343: the loss is taken every loss_every steps;
  // between samples, with nothing downloaded, the step does not block.
  float sampled = 0.0f;
  float* effective_loss = nullptr;
  lcAttentionIoPolicy effective = *policy;
  if (loss_out != nullptr) {
    const int every = resolveLossEvery(session->shape, *policy);
    if (session->train_step_count % static_cast<std::size_t>(every) == 0) {
      effective_loss = &sampled;
    } else if (!policy->download_out && !policy->download_v) {
      effective.synchronize = 0;
    }
  }
  st = attentionTrainResident(ctx, session->res, session->shape, q, k, v, target, out, learning_rate, effective_loss,
                              effective);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  if (loss_out != nullptr) {
    if (effective_loss != nullptr) {
      session->last_loss = sampled;
      session->has_last_loss = true;
      *loss_out = sampled;
    } else {
      *loss_out = session->has_last_loss ? session->last_loss : 0.0f;
    }
  }
  ++session->train_step_count;
  return LC_SUCCESS;
}

lcError_t lcAttentionSessionTrainRunCached(lcAttentionSession* session, float learning_rate, size_t repeat_count) {
  if (session == nullptr || repeat_count == 0 || !(learning_rate > 0.0f)) {
    return toLc(fail(Status::kInvalidValue, "attention session: null session, zero repeat or learning_rate <= 0"));
  }
  HipContext* ctx = nullptr;
  Status st = requireHip(session->device, "attention session train step", &ctx);
  if (st != Status::kSuccess) {
    return toLc(st);
  }
  lcAttentionIoPolicy p = session->default_policy;
  p.upload_q = p.upload_k = p.upload_v = p.upload_target = 0;
  p.download_out = p.download_v = 0;
  p.synchronize = 0;
  std::lock_guard<std::recursive_mutex> lock(ctx->mu);
  // Resident tensors only: nothing is uploaded or downloaded, so the host
  // pointers the step's argument checks require are never read or written.
  float unused = 0.0f;
  for (std::size_t i = 0; i < repeat_count; ++i) {
    st = attentionTrainResident(ctx, session->res, session->shape, &unused, &unused, &unused, &unused, &unused,
                                learning_rate, nullptr, p);
    if (st != Status::kSuccess) {
      return toLc(st);
    }
    ++session->train_step_count;
  }
  return toLc(syncStream(ctx));
}

lcError_t lcAttentionSessionTrainStep(lcAttentionSession* session, const float* q, const float* k, float* v,
                                      const float* target, float* out, float learning_rate, float* loss_out) {
  if (session == nullptr) {
    return toLc(fail(Status::kInvalidValue, "attention session: null session"));
  }
  return lcAttentionSessionTrainStepWithPolicy(session, q, k, v, target, out, learning_rate, loss_out,
                                               &session->default_policy);
}

}  // extern "C"
