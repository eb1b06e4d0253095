/*
 * oracle.c -- CPU restatement of Lightning Core's dense forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker and the CPU baseline.  The product
 * library never links or calls this file.  See oracle.h for what each
 * function restates and what pins it.
 *
 * Built with the reference's Release flags (-O3 -ffast-math -funroll-loops,
 * reference CMakeLists.txt:108-110) by oracle/Makefile.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* src/attention_cpu.cpp:15-36 (dotFloat, non-NEON branch): sequential sum. */
static float orc_dot(const float* a, const float* b, size_t n) {
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    sum += a[i] * b[i];
  }
  return sum;
}

/* src/attention_cpu.cpp:38-101, restricted to query rows [r0, r1).
 * Pass 1 (:53-63) scores with the -1e30f causal mask, pass 2 (:65-82) row
 * softmax (max, exp(s - max), sum, multiply by 1/sum), pass 3 (:84-94) the
 * i -> j -> c accumulation of P.V into a zero-filled output. */
int orc_attention_forward_rows(const float* q, const float* k, const float* v, float* out,
                               size_t s, size_t d, int causal, size_t r0, size_t r1) {
  if (q == NULL || k == NULL || v == NULL || out == NULL || s == 0 || d == 0 || r0 > r1 || r1 > s) {
    return ORC_INVALID_VALUE;
  }
  const size_t rows = r1 - r0;
  if (rows == 0) {
    return ORC_SUCCESS;
  }
  float* scores = (float*)malloc(rows * s * sizeof(float));
  float* probs = (float*)malloc(rows * s * sizeof(float));
  if (scores == NULL || probs == NULL) {
    free(scores);
    free(probs);
    return ORC_OUT_OF_MEMORY;
  }
  const float scale = 1.0f / sqrtf((float)d);

  for (size_t r = 0; r < rows; ++r) {
    const size_t i = r0 + r;
    const float* qi = q + i * d;
    for (size_t j = 0; j < s; ++j) {
      if (causal && j > i) {
        scores[r * s + j] = -1e30f;
      } else {
        scores[r * s + j] = orc_dot(qi, k + j * d, d) * scale;
      }
    }
  }

  for (size_t r = 0; r < rows; ++r) {
    float row_max = scores[r * s];
    for (size_t j = 1; j < s; ++j) {
      row_max = fmaxf(row_max, scores[r * s + j]);
    }
    float row_sum = 0.0f;
    for (size_t j = 0; j < s; ++j) {
      const float e = expf(scores[r * s + j] - row_max);
      probs[r * s + j] = e;
      row_sum += e;
    }
    const float inv = 1.0f / row_sum;
    for (size_t j = 0; j < s; ++j) {
      probs[r * s + j] *= inv;
    }
  }

  memset(out, 0, rows * d * sizeof(float));
  for (size_t r = 0; r < rows; ++r) {
    float* oi = out + r * d;
    for (size_t j = 0; j < s; ++j) {
      const float p = probs[r * s + j];
      const float* vj = v + j * d;
      for (size_t c = 0; c < d; ++c) {
        oi[c] += p * vj[c];
      }
    }
  }

  free(scores);
  free(probs);
  return ORC_SUCCESS;
}

/* src/attention_cpu.cpp:105-112 (attentionForwardCpu -> computeAttentionForward). */
int orc_attention_forward(const float* q, const float* k, const float* v, float* out,
                          size_t s, size_t d, int causal) {
  return orc_attention_forward_rows(q, k, v, out, s, d, causal, 0, s);
}

/* src/attention.cpp:41-60 (applyForwardPostprocess): identity policy is a
 * no-op; otherwise out = out*scale + bias, clamped at 0 when relu. */
void orc_attention_postprocess(float* out, size_t n, float scale, float bias, int relu) {
  if (out == NULL) {
    return;
  }
  if (scale == 1.0f && bias == 0.0f && !relu) {
    return;
  }
  for (size_t i = 0; i < n; ++i) {
    float v = out[i] * scale + bias;
    if (relu && v < 0.0f) {
      v = 0.0f;
    }
    out[i] = v;
  }
}

int orc_attention_forward_batched(const float* q, const float* k, const float* v, float* out,
                                  size_t batch, size_t heads, size_t s, size_t d, int causal) {
  const size_t per = s * d;
  for (size_t bh = 0; bh < batch * heads; ++bh) {
    int st = orc_attention_forward(q + bh * per, k + bh * per, v + bh * per, out + bh * per, s, d, causal);
    if (st != ORC_SUCCESS) {
      return st;
    }
  }
  return ORC_SUCCESS;
}

/* src/attention_cpu.cpp:114-163 (attentionTrainStepCpu): the forward of
 * computeAttentionForward keeping the probabilities P [s, s] (same three
 * passes as orc_attention_forward_rows), then
 *   diff = out - target; loss += diff*diff (sequential, fp32);
 *   grad_out = 2*diff*norm with norm = 1/(s*d);
 *   grad_v[j, c] += P[i, j] * grad_out[i, c]  (j outer, i, c inner);
 *   v -= learning_rate * grad_v;  loss_out = loss * norm.
 * No forward postprocess (the reference applies it only in
 * attentionForwardWithPolicy).  v is updated in place. */
int orc_attention_train_step(const float* q, const float* k, float* v, const float* target, float* out,
                             size_t s, size_t d, int causal, float learning_rate, float* loss_out) {
  if (q == NULL || k == NULL || v == NULL || target == NULL || out == NULL || s == 0 || d == 0) {
    return ORC_INVALID_VALUE;
  }
  float* probs = (float*)malloc(s * s * sizeof(float));
  float* grad_out = (float*)calloc(s * d, sizeof(float));
  float* grad_v = (float*)calloc(s * d, sizeof(float));
  if (probs == NULL || grad_out == NULL || grad_v == NULL) {
    free(probs);
    free(grad_out);
    free(grad_v);
    return ORC_OUT_OF_MEMORY;
  }
  const float scale = 1.0f / sqrtf((float)d);
  for (size_t i = 0; i < s; ++i) {
    for (size_t j = 0; j < s; ++j) {
      probs[i * s + j] = (causal && j > i) ? -1e30f : orc_dot(q + i * d, k + j * d, d) * scale;
    }
  }
  for (size_t i = 0; i < s; ++i) {
    float* row = probs + i * s;
    float row_max = row[0];
    for (size_t j = 1; j < s; ++j) {
      row_max = fmaxf(row_max, row[j]);
    }
    float row_sum = 0.0f;
    for (size_t j = 0; j < s; ++j) {
      row[j] = expf(row[j] - row_max);
      row_sum += row[j];
    }
    const float inv = 1.0f / row_sum;
    for (size_t j = 0; j < s; ++j) {
      row[j] *= inv;
    }
  }
  memset(out, 0, s * d * sizeof(float));
  for (size_t i = 0; i < s; ++i) {
    float* oi = out + i * d;
    for (size_t j = 0; j < s; ++j) {
      const float p = probs[i * s + j];
      const float* vj = v + j * d;
      for (size_t c = 0; c < d; ++c) {
        oi[c] += p * vj[c];
      }
    }
  }
  float loss = 0.0f;
  const float norm = 1.0f / (float)(s * d);
  for (size_t i = 0; i < s * d; ++i) {
    const float diff = out[i] - target[i];
    loss += diff * diff;
    grad_out[i] = 2.0f * diff * norm;
  }
  for (size_t j = 0; j < s; ++j) {
    float* gv = grad_v + j * d;
    for (size_t i = 0; i < s; ++i) {
      const float p = probs[i * s + j];
      const float* go = grad_out + i * d;
      for (size_t c = 0; c < d; ++c) {
        gv[c] += p * go[c];
      }
    }
  }
  for (size_t i = 0; i < s * d; ++i) {
    v[i] -= learning_rate * grad_v[i];
  }
  if (loss_out != NULL) {
    *loss_out = loss * norm;
  }
  free(probs);
  free(grad_out);
  free(grad_v);
  return ORC_SUCCESS;
}

/* src/ops/matmul_cpu.cpp:49-60 (non-Apple branch) for rows [r0, r1):
 * zero-fill, then for i, for p: a = A[i,p]; for j: C[i,j] += a * B[p,j]. */
int orc_matmul_rows(const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                    size_t r0, size_t r1) {
  if (a == NULL || b == NULL || out == NULL || m == 0 || k == 0 || n == 0 || r0 > r1 || r1 > m) {
    return ORC_INVALID_VALUE;
  }
  memset(out, 0, (r1 - r0) * n * sizeof(float));
  for (size_t i = r0; i < r1; ++i) {
    float* orow = out + (i - r0) * n;
    for (size_t p = 0; p < k; ++p) {
      const float av = a[i * k + p];
      const float* brow = b + p * n;
      for (size_t j = 0; j < n; ++j) {
        orow[j] += av * brow[j];
      }
    }
  }
  return ORC_SUCCESS;
}

/* src/ops/matmul_cpu.cpp:12-61 (matMulCpu<float>). */
int orc_matmul(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) {
  return orc_matmul_rows(a, b, out, m, k, n, 0, m);
}

/* core/ops.hpp:855-1213, generic path.  Geometry :886-892; validation
 * :875-884; im2col with zero padding :1149-1177 (row = (n*oh + oy)*ow + ox,
 * col = (c*kh + ky)*kw + kx); packed weights w_col[col, oc] = w[oc, col]
 * (:1044-1095); out2d = cols . w_col via matMul (:1184-1192); scatter back to
 * NCHW with bias and optional ReLU (:1197-1210). */
int orc_conv2d_nchw(const float* x, const float* w, const float* bias, float* out,
                    size_t batch, size_t in_c, size_t in_h, size_t in_w,
                    size_t out_c, size_t kh, size_t kw,
                    size_t sh, size_t sw, size_t ph, size_t pw, int relu) {
  if (x == NULL || w == NULL || out == NULL || batch == 0 || in_c == 0 || in_h == 0 || in_w == 0 ||
      out_c == 0 || kh == 0 || kw == 0 || sh == 0 || sw == 0) {
    return ORC_INVALID_VALUE;
  }
  if (in_h + 2 * ph < kh || in_w + 2 * pw < kw) {
    return ORC_INVALID_VALUE;
  }
  const size_t out_h = (in_h + 2 * ph - kh) / sh + 1;
  const size_t out_w = (in_w + 2 * pw - kw) / sw + 1;
  const size_t kin = in_c * kh * kw;
  const size_t rows = batch * out_h * out_w;

  float* cols = (float*)calloc(rows * kin, sizeof(float));
  float* w_col = (float*)malloc(kin * out_c * sizeof(float));
  float* out2d = (float*)malloc(rows * out_c * sizeof(float));
  if (cols == NULL || w_col == NULL || out2d == NULL) {
    free(cols);
    free(w_col);
    free(out2d);
    return ORC_OUT_OF_MEMORY;
  }

  for (size_t oc = 0; oc < out_c; ++oc) {
    for (size_t col = 0; col < kin; ++col) {
      w_col[col * out_c + oc] = w[oc * kin + col];
    }
  }

  for (size_t nb = 0; nb < batch; ++nb) {
    for (size_t oy = 0; oy < out_h; ++oy) {
      for (size_t ox = 0; ox < out_w; ++ox) {
        const size_t row = (nb * out_h + oy) * out_w + ox;
        for (size_t c = 0; c < in_c; ++c) {
          for (size_t ky = 0; ky < kh; ++ky) {
            const size_t y_nom = oy * sh + ky;
            if (y_nom < ph || y_nom - ph >= in_h) {
              continue;
            }
            for (size_t kx = 0; kx < kw; ++kx) {
              const size_t x_nom = ox * sw + kx;
              if (x_nom < pw || x_nom - pw >= in_w) {
                continue;
              }
              const size_t col = (c * kh + ky) * kw + kx;
              cols[row * kin + col] = x[((nb * in_c + c) * in_h + (y_nom - ph)) * in_w + (x_nom - pw)];
            }
          }
        }
      }
    }
  }

  int st = orc_matmul(cols, w_col, out2d, rows, kin, out_c);
  if (st == ORC_SUCCESS) {
    for (size_t nb = 0; nb < batch; ++nb) {
      for (size_t oy = 0; oy < out_h; ++oy) {
        for (size_t ox = 0; ox < out_w; ++ox) {
          const size_t row = (nb * out_h + oy) * out_w + ox;
          for (size_t oc = 0; oc < out_c; ++oc) {
            float v = out2d[row * out_c + oc] + (bias != NULL ? bias[oc] : 0.0f);
            if (relu && v < 0.0f) {
              v = 0.0f;
            }
            out[((nb * out_c + oc) * out_h + oy) * out_w + ox] = v;
          }
        }
      }
    }
  }
  free(cols);
  free(w_col);
  free(out2d);
  return st;
}

/* python/bindings/bind_integrated.cpp:709-729: copy min(conv_size, total),
 * then double the filled prefix until 3*need floats are filled. */
void orc_qkv_pack_repeat(const float* conv, size_t conv_size, size_t need, float* packed) {
  const size_t total = need * 3;
  size_t copied = conv_size < total ? conv_size : total;
  memcpy(packed, conv, copied * sizeof(float));
  while (copied < total) {
    const size_t chunk = copied < (total - copied) ? copied : (total - copied);
    memcpy(packed + copied, packed, chunk * sizeof(float));
    copied += chunk;
  }
}

/* python/bindings/bind_integrated.cpp:614-730 (eager mode). */
int orc_conv_attention_torchstrong_nchw(const float* x, const float* w, const float* bias, float* out,
                                        size_t batch, size_t in_c, size_t in_h, size_t in_w,
                                        size_t out_c, size_t kh, size_t kw,
                                        size_t seq_len, size_t head_dim,
                                        size_t sh, size_t sw, size_t ph, size_t pw) {
  if (sh == 0 || sw == 0 || in_h + 2 * ph < kh || in_w + 2 * pw < kw || seq_len == 0 || head_dim == 0) {
    return ORC_INVALID_VALUE;
  }
  const size_t out_h = (in_h + 2 * ph - kh) / sh + 1;
  const size_t out_w = (in_w + 2 * pw - kw) / sw + 1;
  const size_t conv_size = batch * out_c * out_h * out_w;
  const size_t need = seq_len * head_dim;
  const size_t total = 3 * need;

  float* conv = (float*)malloc(conv_size * sizeof(float));
  float* packed = (float*)malloc(total * sizeof(float));
  if (conv == NULL || packed == NULL) {
    free(conv);
    free(packed);
    return ORC_OUT_OF_MEMORY;
  }
  int st = orc_conv2d_nchw(x, w, bias, conv, batch, in_c, in_h, in_w, out_c, kh, kw, sh, sw, ph, pw, 1);
  if (st == ORC_SUCCESS) {
    const float* src = conv;
    if (conv_size < total) {
      orc_qkv_pack_repeat(conv, conv_size, need, packed);
      src = packed;
    }
    st = orc_attention_forward(src, src + need, src + 2 * need, out, seq_len, head_dim, 0);
  }
  free(conv);
  free(packed);
  return st;
}

int orc_vit_block(const float* x, const float* w_conv, const float* w_qkv, const float* w_o, float* out,
                  size_t batch, size_t in_c, size_t img_h, size_t img_w, size_t patch,
                  size_t embed, size_t heads, size_t row_begin, size_t row_end) {
  if (x == NULL || w_conv == NULL || w_qkv == NULL || w_o == NULL || out == NULL || patch == 0 ||
      heads == 0 || embed % heads != 0 || img_h < patch || img_w < patch) {
    return ORC_INVALID_VALUE;
  }
  const size_t gh = (img_h - patch) / patch + 1;
  const size_t gw = (img_w - patch) / patch + 1;
  const size_t t_len = gh * gw;
  const size_t dh = embed / heads;
  if (row_begin > row_end || row_end > batch * t_len) {
    return ORC_INVALID_VALUE;
  }

  float* conv = (float*)malloc(embed * t_len * sizeof(float));
  float* tokens = (float*)malloc(t_len * embed * sizeof(float));
  float* qkv = (float*)malloc(t_len * 3 * embed * sizeof(float));
  float* qh = (float*)malloc(t_len * dh * sizeof(float));
  float* kh = (float*)malloc(t_len * dh * sizeof(float));
  float* vh = (float*)malloc(t_len * dh * sizeof(float));
  float* oh = (float*)malloc(t_len * dh * sizeof(float));
  float* attn = (float*)malloc(t_len * embed * sizeof(float));
  int st = ORC_SUCCESS;
  if (!conv || !tokens || !qkv || !qh || !kh || !vh || !oh || !attn) {
    st = ORC_OUT_OF_MEMORY;
  }

  for (size_t b = 0; st == ORC_SUCCESS && b < batch; ++b) {
    const size_t img_r0 = b * t_len;
    const size_t img_r1 = img_r0 + t_len;
    const size_t lo = row_begin > img_r0 ? row_begin : img_r0;
    const size_t hi = row_end < img_r1 ? row_end : img_r1;
    if (lo >= hi) {
      continue;
    }
    const size_t t0 = lo - img_r0;
    const size_t t1 = hi - img_r0;

    st = orc_conv2d_nchw(x + b * in_c * img_h * img_w, w_conv, NULL, conv, 1, in_c, img_h, img_w, embed,
                         patch, patch, patch, patch, 0, 0, 1);
    if (st != ORC_SUCCESS) {
      break;
    }
    for (size_t t = 0; t < t_len; ++t) {
      for (size_t c = 0; c < embed; ++c) {
        tokens[t * embed + c] = conv[c * t_len + t];
      }
    }
    st = orc_matmul(tokens, w_qkv, qkv, t_len, embed, 3 * embed);
    if (st != ORC_SUCCESS) {
      break;
    }
    for (size_t h = 0; h < heads && st == ORC_SUCCESS; ++h) {
      for (size_t t = 0; t < t_len; ++t) {
        for (size_t dd = 0; dd < dh; ++dd) {
          qh[t * dh + dd] = qkv[t * 3 * embed + 0 * embed + h * dh + dd];
          kh[t * dh + dd] = qkv[t * 3 * embed + 1 * embed + h * dh + dd];
          vh[t * dh + dd] = qkv[t * 3 * embed + 2 * embed + h * dh + dd];
        }
      }
      st = orc_attention_forward_rows(qh, kh, vh, oh, t_len, dh, 0, t0, t1);
      for (size_t t = t0; t < t1; ++t) {
        for (size_t dd = 0; dd < dh; ++dd) {
          attn[t * embed + h * dh + dd] = oh[(t - t0) * dh + dd];
        }
      }
    }
    if (st != ORC_SUCCESS) {
      break;
    }
    st = orc_matmul_rows(attn, w_o, out + (lo - row_begin) * embed, t_len, embed, embed, t0, t1);
  }

  free(conv);
  free(tokens);
  free(qkv);
  free(qh);
  free(kh);
  free(vh);
  free(oh);
  free(attn);
  return st;
}
