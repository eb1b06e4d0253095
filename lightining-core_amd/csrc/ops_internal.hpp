// ops_internal.hpp -- device-side state shared by the op front-ends.
#pragma once

#include "kernels.hpp"
#include "lc_internal.hpp"

namespace lchip {

inline bool isHalf(lcDataType t) { return t == LC_DTYPE_BF16 || t == LC_DTYPE_F16; }
inline kern::Half halfOf(lcDataType t) { return t == LC_DTYPE_F16 ? kern::Half::kF16 : kern::Half::kBF16; }
inline bool validDtype(lcDataType t) { return t == LC_DTYPE_F32 || t == LC_DTYPE_BF16 || t == LC_DTYPE_F16; }

// Shape of an attention problem: batch*heads independent [S, D] problems.
struct AttnShape {
  std::size_t batch = 1;
  std::size_t heads = 1;
  std::size_t seq_len = 0;
  std::size_t head_dim = 0;
  bool causal = false;
  lcDataType dtype = LC_DTYPE_F32;
  std::size_t bh() const { return batch * heads; }
  std::size_t elems() const { return bh() * seq_len * head_dim; }
  std::size_t sPad() const { return roundUp(seq_len, kern::kAttnQBlock); }
};

// Device buffers of one attention problem.  fp32 path: q/k/v/out [BH, S, D].
// 16-bit path: q/k [BH, S_pad, D] and vt [BH, D, S_pad] (zero padded),
// out fp32 [BH, S, D], stage = fp32 upload staging.
// Train step (fp32, one head): target [S, D], stats [S, 2] (softmax m, l of
// the forward), loss one float.
struct AttnResident {
  AttnShape shape;
  DeviceBuffer q, k, v, out, stage;
  DeviceBuffer target, stats, loss;
  DeviceBuffer v_scratch;  // the train step's dV autotune runs on a copy of V
  DeviceBuffer split_ws;   // partials of the fp32 forward's key splits
  bool has_q = false, has_k = false, has_v = false, has_out = false, has_target = false;
};

// Runs one forward on `res` with the reference's policy semantics.
// Host pointers may be null where the policy does not use them.
Status attentionForwardResident(HipContext* ctx, AttnResident& res, const AttnShape& shape, const float* q,
                                const float* k, const float* v, float* out, const lcAttentionIoPolicy& policy,
                                std::size_t repeat);

// One attention train step on `res` (reference attentionTrainStepWithPolicy,
// src/attention.cpp:217-244, CPU semantics of attention_cpu.cpp:114-163):
// forward, loss (when loss_out != nullptr), V -= lr * dV in the resident V,
// downloads per policy.
Status attentionTrainResident(HipContext* ctx, AttnResident& res, const AttnShape& shape, const float* q,
                              const float* k, float* v, const float* target, float* out, float learning_rate,
                              float* loss_out, const lcAttentionIoPolicy& policy);

// Device buffers of one GEMM, zero padded to the kernel tiles.  fp32:
// a [roundup(M,64), roundup(K,64)], b [roundup(K,64), roundup(N,64)];
// 16-bit: a [roundup(M,256), roundup(K,64)], bt [roundup(N,256), roundup(K,64)];
// c fp32 [M,N]; stage fp32 upload staging.
struct MatMulResident {
  std::size_t m = 0, k = 0, n = 0;
  lcDataType dtype = LC_DTYPE_F32;
  DeviceBuffer a, b, c, stage;
  bool has_a = false, has_b = false, has_c = false;
  // GEMM kernel variant for this shape (kern::GemmF32Variant or
  // kern::GemmHalfVariant as int; 0 = the launcher's own choice), settled on
  // the first launch from the tune cache, an autotune or the heuristic.
  int variant = 0;
  bool tuned = false;
};

Status matmulResident(HipContext* ctx, MatMulResident& res, std::size_t m, std::size_t k, std::size_t n,
                      lcDataType dtype, const float* a, const float* b, float* out, const lcMatMulIoPolicy& policy,
                      std::size_t repeat);

// Validation helpers returning kInvalidValue with a message.
Status requireHip(lcDeviceKind device, const char* op, HipContext** ctx_out);

}  // namespace lchip
