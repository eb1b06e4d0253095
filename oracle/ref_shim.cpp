// ref_shim.cpp -- C entry points over the reference's own CPU path, compiled
// from the reference sources where they lie (see oracle/Makefile).  TEST
// INFRASTRUCTURE ONLY: used to write tests/golden fixtures and, optionally, as
// bench.py's CPU baseline.  Never linked into the product library.
//
// Calls (reference file:line):
//   lightning_core::attentionForwardWithPolicy   src/attention.cpp:137-201
//   lightning_core::attentionTrainStep           src/attention.cpp:203-214
//   lightning_core::ops::matMul<float>           include/lightning_core/core/ops.hpp:195-205
//   lightning_core::ops::conv2dNchw<float>       include/lightning_core/core/ops.hpp:855-1213
// all with Device::kCPU.
#include <cstring>
#include <vector>

#include "lightning_core/core/attention.hpp"
#include "lightning_core/core/ops.hpp"

namespace lc = lightning_core;

extern "C" {

int ref_attention_forward(const float* q, const float* k, const float* v, float* out, size_t s, size_t d,
                          int causal, float out_scale, float out_bias, int out_relu) {
  lc::AttentionConfig cfg{s, d, causal != 0};
  lc::AttentionIoPolicy policy;
  policy.output_scale = out_scale;
  policy.output_bias = out_bias;
  policy.output_relu = out_relu != 0;
  return static_cast<int>(lc::attentionForwardWithPolicy(q, k, v, out, cfg, lc::runtime::Device::kCPU, policy));
}

// attentionTrainStep (src/attention.cpp:203-214) on the CPU device: v is
// updated in place, *loss receives the mean squared error.
int ref_attention_train_step(const float* q, const float* k, float* v, const float* target, float* out, size_t s,
                             size_t d, int causal, float learning_rate, float* loss) {
  lc::AttentionConfig cfg{s, d, causal != 0};
  return static_cast<int>(
      lc::attentionTrainStep(q, k, v, target, out, learning_rate, cfg, lc::runtime::Device::kCPU, loss));
}

int ref_matmul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) {
  return static_cast<int>(lc::ops::matMul<float>(a, b, out, m, k, n, lc::runtime::Device::kCPU));
}

int ref_conv2d_nchw(const float* x, const float* w, const float* bias, float* out, size_t batch, size_t in_c,
                    size_t in_h, size_t in_w, size_t out_c, size_t kh, size_t kw, size_t sh, size_t sw,
                    size_t ph, size_t pw, int relu) {
  return static_cast<int>(lc::ops::conv2dNchw<float>(x, w, bias, out, batch, in_c, in_h, in_w, out_c, kh, kw, sh,
                                                     sw, ph, pw, lc::runtime::Device::kCPU, relu != 0));
}

// The reference's conv->attention chain (bind_integrated.cpp:614-730) lives in
// a pybind translation unit; this composes the same steps from the reference's
// conv2dNchw and attentionForward with the flat-slice / repeat packing.
int ref_conv_attention(const float* x, const float* w, const float* bias, float* out, size_t batch, size_t in_c,
                       size_t in_h, size_t in_w, size_t out_c, size_t kh, size_t kw, size_t seq_len,
                       size_t head_dim, size_t sh, size_t sw, size_t ph, size_t pw) {
  const size_t out_h = (in_h + 2 * ph - kh) / sh + 1;
  const size_t out_w = (in_w + 2 * pw - kw) / sw + 1;
  const size_t conv_size = batch * out_c * out_h * out_w;
  std::vector<float> conv(conv_size);
  int st = ref_conv2d_nchw(x, w, bias, conv.data(), batch, in_c, in_h, in_w, out_c, kh, kw, sh, sw, ph, pw, 1);
  if (st != 0) {
    return st;
  }
  const size_t need = seq_len * head_dim;
  const size_t total = 3 * need;
  std::vector<float> packed(total);
  size_t copied = conv_size < total ? conv_size : total;
  std::memcpy(packed.data(), conv.data(), copied * sizeof(float));
  while (copied < total) {
    const size_t chunk = copied < total - copied ? copied : total - copied;
    std::memcpy(packed.data() + copied, packed.data(), chunk * sizeof(float));
    copied += chunk;
  }
  lc::AttentionConfig cfg{seq_len, head_dim, false};
  return static_cast<int>(lc::attentionForward(packed.data(), packed.data() + need, packed.data() + 2 * need, out,
                                               cfg, lc::runtime::Device::kCPU));
}

}  // extern "C"
