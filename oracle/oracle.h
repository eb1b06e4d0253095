/*
 * oracle.h -- CPU restatement of Lightning Core's dense forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / CPU baseline.
 *
 * Every function restates one reference function (file:line under the
 * reference tree); the restatement is written fresh in C and keeps the
 * reference's pass order, constants and accumulation order:
 *   - attention: three passes (scores, row softmax, P.V), -1e30f causal mask,
 *     scale = 1/sqrtf(D), exp(s - rowmax), multiply by 1/rowsum;
 *   - matmul: zero-fill then the i-p-j loop with fp32 accumulation;
 *   - conv2d: im2col (col = (c*kh + ky)*kw + kx) + matmul + bias/ReLU scatter;
 *   - QkvPackRepeat: consecutive S*D slices of the flat conv output, tiled by
 *     repetition when the conv output is shorter than 3*S*D.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   orc_attention_forward      golden vectors from the compiled reference
 *                              (tests/golden), 2x2 KAT, fp64 brute force,
 *                              softmax invariants (constant V, causal row 0,
 *                              q = 0 -> column mean of V)
 *   orc_attention_postprocess  closed form + golden vector
 *   orc_attention_train_step   golden vectors from the compiled reference,
 *                              fp64 recomputation of loss / grad_v / update,
 *                              closed form (V = target-free uniform case)
 *   orc_matmul                 golden vectors, 2x3.3x2 KAT, fp64 brute force
 *   orc_conv2d_nchw            golden vectors, direct-convolution brute force
 *   orc_qkv_pack_repeat        golden vector (conv->attention), closed form
 *                              (numpy.resize tiling)
 *   orc_conv_attention_torchstrong_nchw  golden vectors
 *   orc_vit_block              independent float64 numpy composition
 *                              (patch-embed conv, timm (B,N,3,H,D) split)
 * Row-subset variants compute a subset of output rows with exactly the same
 * arithmetic as the full functions (rows are independent); tests check that.
 */
#ifndef LC_ORACLE_H
#define LC_ORACLE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status values mirror lightning_core::runtime::Status (runtime.hpp:24-32). */
enum { ORC_SUCCESS = 0, ORC_INVALID_VALUE = 2, ORC_OUT_OF_MEMORY = 3 };

/* src/attention_cpu.cpp:38-101 (computeAttentionForward), q/k/v/out [s, d]. */
int orc_attention_forward(const float* q, const float* k, const float* v, float* out,
                          size_t s, size_t d, int causal);

/* Same arithmetic restricted to query rows [row_begin, row_end); out holds
 * (row_end - row_begin) rows of d floats. */
int orc_attention_forward_rows(const float* q, const float* k, const float* v, float* out,
                               size_t s, size_t d, int causal, size_t row_begin, size_t row_end);

/* src/attention.cpp:41-60 (applyForwardPostprocess). */
void orc_attention_postprocess(float* out, size_t n, float scale, float bias, int relu);

/* orc_attention_forward applied to each of batch*heads contiguous [s, d]
 * problems (layout [batch, heads, s, d]). */
int orc_attention_forward_batched(const float* q, const float* k, const float* v, float* out,
                                  size_t batch, size_t heads, size_t s, size_t d, int causal);

/* src/attention_cpu.cpp:114-163 (attentionTrainStepCpu): forward (out),
 * mean-squared-error loss against target, grad_v = P^T . grad_out, SGD update
 * of v in place; *loss_out (if not NULL) = mean of (out - target)^2. */
int orc_attention_train_step(const float* q, const float* k, float* v, const float* target, float* out,
                             size_t s, size_t d, int causal, float learning_rate, float* loss_out);

/* src/ops/matmul_cpu.cpp:49-60 (matMulCpu, non-Apple branch). */
int orc_matmul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n);

/* Rows [row_begin, row_end) of orc_matmul; out holds those rows. */
int orc_matmul_rows(const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                    size_t row_begin, size_t row_end);

/* core/ops.hpp:855-1213 (ops::conv2dNchw<float>, generic im2col path:
 * im2col :1149-1177, packed weights :1044-1095, matmul :1184-1192, bias/ReLU
 * scatter :1197-1210).  x [batch, in_c, in_h, in_w], w [out_c, in_c, kh, kw],
 * bias [out_c] or NULL, out [batch, out_c, out_h, out_w]. */
int orc_conv2d_nchw(const float* x, const float* w, const float* bias, float* out,
                    size_t batch, size_t in_c, size_t in_h, size_t in_w,
                    size_t out_c, size_t kh, size_t kw,
                    size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w, int relu);

/* python/bindings/bind_integrated.cpp:709-729 (QkvPackRepeat): packed holds
 * 3*need floats; the first conv_size are the conv output, the rest repeat it. */
void orc_qkv_pack_repeat(const float* conv, size_t conv_size, size_t need, float* packed);

/* python/bindings/bind_integrated.cpp:614-730
 * (convAttentionTorchstrongNchwIntoDirect): conv2d + ReLU (+bias), then Q/K/V
 * = consecutive seq_len*head_dim slices of the flat NCHW output (repeated if
 * short), then single-head non-causal attention.  out [seq_len, head_dim]. */
int orc_conv_attention_torchstrong_nchw(const float* x, const float* w, const float* bias, float* out,
                                        size_t batch, size_t in_c, size_t in_h, size_t in_w,
                                        size_t out_c, size_t kh, size_t kw,
                                        size_t seq_len, size_t head_dim,
                                        size_t stride_h, size_t stride_w, size_t pad_h, size_t pad_w);

/* ViT-style block composed from the functions above (the reference has the
 * pieces but not this composition):
 *   conv = relu(conv2d_nchw(x, w_conv, stride = patch, pad = 0))      [B, E, g, g]
 *   tokens[b, t, c] = conv[b, c, t / g, t % g]                         [B, T, E]
 *   qkv = tokens . w_qkv           (w_qkv [E, 3E], matmul_cpu)          [B, T, 3E]
 *   q/k/v[b, h, t, dd] = qkv[b, t, which*E + h*Dh + dd]  (timm order)
 *   attn[b, t, h*Dh + dd] = attention_forward(q[b,h], k[b,h], v[b,h])   non-causal
 *   out = attn . w_o               (w_o [E, E])                          [B, T, E]
 * Only output rows (b, t) with b*T + t in [row_begin, row_end) are written
 * (row_begin = 0, row_end = B*T for the full block); out holds those rows. */
int orc_vit_block(const float* x, const float* w_conv, const float* w_qkv, const float* w_o, float* out,
                  size_t batch, size_t in_c, size_t img_h, size_t img_w, size_t patch,
                  size_t embed, size_t heads, size_t row_begin, size_t row_end);

#ifdef __cplusplus
}
#endif

#endif /* LC_ORACLE_H */
