// attention.hip -- flash-style attention forward on gfx950 MFMA.
//
// Formulation (both kernels).  Each wave owns 32 queries.  Scores are computed
// transposed, S^T = K . Q^T, so lane l holds the scores of ONE query (l % 32)
// against 16 keys of every 32-key tile (the other 16 sit in lane l ^ 32).
// The row max therefore needs one cross-lane step (lane ^ 32) and the running
// sum none until the end.  The output is also accumulated transposed,
// O^T = V^T . P^T, whose B operand is P^T: exactly the probabilities the lane
// already holds in its score registers (the key order inside an MFMA k-block
// is a free permutation shared by both operands), so P never leaves the
// registers and O's rows line up with the lane's softmax statistics (the
// rescale by exp(m_old - m_new) is a per-lane multiply).
//
// Softmax follows the reference's arithmetic (src/attention_cpu.cpp:38-101):
// s = (q.k) * (1/sqrt(D)), masked entries -1e30 (causal j > i, plus padding
// keys j >= S), p = exp(s - max), out = sum p v / sum p; the exponentials are
// evaluated as exp2 with log2(e) folded into the scale (online form).
#include <math.h>

#include "../kernels.hpp"
#include "kcommon.hpp"

namespace lchip::k {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaskValue = -1e30f;

// ---------------------------------------------------------------------------
// fp32: one wave per 32 queries, 32-key tiles in LDS, v_mfma_f32_32x32x2_f32.
// D padded to 32*DT (zeros).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(64) void attn_fwd_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, float* __restrict__ out,
                                                          int S, int D, int causal, float scale, float post_scale,
                                                          float post_bias, int post_relu) {
  constexpr int DP = 32 * DT;
  __shared__ float Qs[32][DP + 1];
  __shared__ float Ks[32][DP + 1];
  __shared__ float Vs[32][DP];
  const int lane = threadIdx.x;
  const int nqb = (S + 31) / 32;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x);  // heaviest (causal) blocks first
  const int q0 = qb * 32;
  const size_t head = static_cast<size_t>(blockIdx.y) * S * D;
  q += head;
  k += head;
  v += head;
  out += head;

  for (int idx = lane; idx < 32 * DP; idx += 64) {
    const int r = idx / DP;
    const int c = idx - r * DP;
    Qs[r][c] = (q0 + r < S && c < D) ? q[static_cast<size_t>(q0 + r) * D + c] : 0.0f;
  }
  const int dsteps = (D + 1) / 2 * 2;  // k-extent of S^T = K . Q^T (zero padded)

  floatx16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    o[t] = zero16();
  }
  float m_run = kMaskValue;
  float l_run = 0.0f;
  const int qi = q0 + (lane & 31);
  const int kend = causal ? min(S, q0 + 32) : S;

  for (int j0 = 0; j0 < kend; j0 += 32) {
    __syncthreads();
    for (int idx = lane; idx < 32 * DP; idx += 64) {
      const int r = idx / DP;
      const int cc = idx - r * DP;
      const bool ok = (j0 + r < S && cc < D);
      Ks[r][cc] = ok ? k[static_cast<size_t>(j0 + r) * D + cc] : 0.0f;
      Vs[r][cc] = ok ? v[static_cast<size_t>(j0 + r) * D + cc] : 0.0f;
    }
    __syncthreads();

    floatx16 st = zero16();
    for (int dd = 0; dd < dsteps; dd += 2) {
      const float a = Ks[lane & 31][dd + (lane >> 5)];
      const float b = Qs[lane & 31][dd + (lane >> 5)];
      st = mfma32x32x2f32(a, b, st);
    }
    float mt = kMaskValue;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = j0 + acc_row(i, lane);
      // (q.k) * scale as the reference, then to the log2 domain
      float x = (st[i] * scale) * kLog2e;
      if (key >= S || (causal && key > qi)) {
        x = kMaskValue;
      }
      st[i] = x;
      mt = fmaxf(mt, x);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = exp2f(m_run - m_new);
    float ls = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = exp2f(st[i] - m_new);
      st[i] = p;
      ls += p;
    }
    l_run = l_run * alpha + ls;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        o[t][i] *= alpha;
      }
    }
    // O^T += V^T . P^T, one key per lane-half per step: key = acc_row(s, lane).
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int kr = acc_row(s, lane);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const float a = Vs[kr][t * 32 + (lane & 31)];
        o[t] = mfma32x32x2f32(a, st[s], o[t]);
      }
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (qi < S) {
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = t * 32 + acc_row(i, lane);
        if (d < D) {
          float val = o[t][i] * inv;
          if (post_scale != 1.0f || post_bias != 0.0f || post_relu) {
            val = val * post_scale + post_bias;
            if (post_relu && val < 0.0f) {
              val = 0.0f;
            }
          }
          out[static_cast<size_t>(qi) * D + d] = val;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 16-bit: 4 waves x 32 queries per workgroup, 64-key tiles.  K tile and V^T
// tile are double-buffered in LDS; the next tile is prefetched into registers
// while the current one is computed, so each tile costs one barrier.  Q
// fragments live in registers; v_mfma_f32_32x32x16_{bf16,f16}.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void attn_fwd_half_kernel(const uint16_t* __restrict__ Q,
                                                               const uint16_t* __restrict__ K,
                                                               const uint16_t* __restrict__ Vt, float* __restrict__ O,
                                                               uint16_t* __restrict__ Ocat, int heads, int S,
                                                               int S_pad, int causal, float scale) {
  constexpr int KT = 64;
  constexpr int LDK = D + 8;
  constexpr int LDV = KT + 8;
  constexpr int DT = D / 32;
  constexpr int QS = D / 16;
  constexpr int KCH = KT * D / 8 / 256;  // 16-byte chunks of the K tile per thread
  constexpr int VCH = D * KT / 8 / 256;  // ... of the V^T tile
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][KT * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][D * LDV];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nqb = S_pad / 128;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.y);  // heaviest (causal) blocks first
  const int bh = blockIdx.x;
  const int q0 = qb * 128 + wave * 32;
  const size_t hoff = static_cast<size_t>(bh) * S_pad * D;
  const uint16_t* Qh = Q + hoff;
  const uint16_t* Kh = K + hoff;
  const uint16_t* Vh = Vt + hoff;
  const int lrow = lane & 31;
  const int half = lane >> 5;

  u32x4 kreg[KCH];
  u32x4 vreg[VCH];
  auto load_tile = [&](int j0) {
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const int ch = c * 256 + tid;
      const int r = ch / (D / 8);
      const int col = (ch - r * (D / 8)) * 8;
      kreg[c] = *reinterpret_cast<const u32x4*>(Kh + static_cast<size_t>(j0 + r) * D + col);
    }
#pragma unroll
    for (int c = 0; c < VCH; ++c) {
      const int ch = c * 256 + tid;
      const int r = ch / (KT / 8);
      const int col = (ch - r * (KT / 8)) * 8;
      vreg[c] = *reinterpret_cast<const u32x4*>(Vh + static_cast<size_t>(r) * S_pad + j0 + col);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const int ch = c * 256 + tid;
      const int r = ch / (D / 8);
      const int col = (ch - r * (D / 8)) * 8;
      *reinterpret_cast<u32x4*>(&Ks[buf][r * LDK + col]) = kreg[c];
    }
#pragma unroll
    for (int c = 0; c < VCH; ++c) {
      const int ch = c * 256 + tid;
      const int r = ch / (KT / 8);
      const int col = (ch - r * (KT / 8)) * 8;
      *reinterpret_cast<u32x4*>(&Vs[buf][r * LDV + col]) = vreg[c];
    }
  };

  u32x4 qf[QS];
#pragma unroll
  for (int s = 0; s < QS; ++s) {
    qf[s] = *reinterpret_cast<const u32x4*>(Qh + static_cast<size_t>(q0 + lrow) * D + s * 16 + 8 * half);
  }
  floatx16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    o[t] = zero16();
  }
  float m_run = kMaskValue;
  float l_run = 0.0f;
  const int qi = q0 + lrow;
  const float c = scale * kLog2e;
  const int kend = causal ? min(S, qb * 128 + 128) : S;

  load_tile(0);
  store_tile(0);
  __syncthreads();
  int buf = 0;
  for (int j0 = 0; j0 < kend; j0 += KT) {
    const bool more = j0 + KT < kend;
    if (more) {
      load_tile(j0 + KT);
    }
    if (!(causal && j0 > q0 + 31)) {  // else every key of the tile follows every query of this wave
      const uint16_t* ks = Ks[buf];
      const uint16_t* vs = Vs[buf];
      floatx16 sc[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        sc[kt] = zero16();
#pragma unroll
        for (int s = 0; s < QS; ++s) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(&ks[(kt * 32 + lrow) * LDK + s * 16 + 8 * half]);
          sc[kt] = mfma32x32x16<T>(a, qf[s], sc[kt]);
        }
      }
      // Raw scores s = q.k; the scale is applied inside the exponent:
      // p = exp2(s*c - m*c) with m the running max of raw scores (c > 0).
      const bool need_mask = (j0 + KT > S) || (causal && j0 + KT - 1 > q0);
      if (need_mask) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = j0 + kt * 32 + acc_row(i, lane);
            if (key >= S || (causal && key > qi)) {
              sc[kt][i] = kMaskValue;
            }
          }
        }
      }
      float mt = kMaskValue;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          mt = fmaxf(mt, sc[kt][i]);
        }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      // Rescale O and l only when some lane's max grew by more than 8/c
      // (exp2 units); otherwise keep the stale reference max.  O and l always
      // share the same reference, so O/l is unchanged; exponents stay <= 8.
      const float m_cand = fmaxf(m_run, mt);
      if (__any((m_cand - m_run) * c > 8.0f)) {
        const float alpha = fast_exp2((m_run - m_cand) * c);
        m_run = m_cand;
        l_run *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            o[t][i] *= alpha;
          }
        }
      }
      const float mc = m_run * c;
      float ls = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = fast_exp2(__builtin_fmaf(sc[kt][i], c, -mc));
          sc[kt][i] = p;
          ls += p;
        }
      }
      l_run += ls;
      // O^T += V^T . P^T over 4 key-steps of 16; element j of step ks is key
      // 16*ks + 8*(j/4) + 4*half + j%4 = accumulator register 8*(ks&1) + j of sc[ks>>1].
#pragma unroll
      for (int ks2 = 0; ks2 < 4; ++ks2) {
        const floatx16& p = sc[ks2 >> 1];
        const int b0 = (ks2 & 1) * 8;
        u32x4 pb;
        pb[0] = pack2<T>(p[b0 + 0], p[b0 + 1]);
        pb[1] = pack2<T>(p[b0 + 2], p[b0 + 3]);
        pb[2] = pack2<T>(p[b0 + 4], p[b0 + 5]);
        pb[3] = pack2<T>(p[b0 + 6], p[b0 + 7]);
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const uint16_t* vp = &vs[(t * 32 + lrow) * LDV + 16 * ks2 + 4 * half];
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vp);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vp + 8);
          const u32x4 va{lo[0], lo[1], hi[0], hi[1]};
          o[t] = mfma32x32x16<T>(va, pb, o[t]);
        }
      }
    }
    if (more) {
      store_tile(buf ^ 1);
    }
    __syncthreads();
    buf ^= 1;
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (qi < S) {
    if (Ocat == nullptr) {
      float* orow = O + (static_cast<size_t>(bh) * S + qi) * D;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = t * 32 + 8 * g + 4 * half;
          const float4 val = make_float4(o[t][4 * g] * inv, o[t][4 * g + 1] * inv, o[t][4 * g + 2] * inv,
                                         o[t][4 * g + 3] * inv);
          *reinterpret_cast<float4*>(orow + d) = val;
        }
      }
    } else {
      const int b = bh / heads;
      const int h = bh - b * heads;
      uint16_t* orow = Ocat + (static_cast<size_t>(b) * S + qi) * (heads * D) + h * D;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = t * 32 + 8 * g + 4 * half;
          u32x2 w;
          w[0] = pack2<T>(o[t][4 * g] * inv, o[t][4 * g + 1] * inv);
          w[1] = pack2<T>(o[t][4 * g + 2] * inv, o[t][4 * g + 3] * inv);
          *reinterpret_cast<u32x2*>(orow + d) = w;
        }
      }
    }
  }
}

}  // namespace lchip::k

namespace lchip::kern {

using namespace lchip::k;

hipError_t attentionF32(const float* q, const float* k, const float* v, float* out, int bh, int S, int D, bool causal,
                        float post_scale, float post_bias, int post_relu, hipStream_t stream) {
  if (D <= 0 || D > 256 || S <= 0 || bh <= 0) {
    return hipErrorInvalidValue;
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(D));
  const dim3 grid((S + 31) / 32, bh);
  const int dt = (D + 31) / 32;
  const int cz = causal ? 1 : 0;
#define LC_ATTN_F32(DT_)                                                                                            \
  hipLaunchKernelGGL((attn_fwd_f32_kernel<DT_>), grid, dim3(64), 0, stream, q, k, v, out, S, D, cz, scale,           \
                     post_scale, post_bias, post_relu)
  switch (dt) {
    case 1: LC_ATTN_F32(1); break;
    case 2: LC_ATTN_F32(2); break;
    case 3: LC_ATTN_F32(3); break;
    case 4: LC_ATTN_F32(4); break;
    case 5: LC_ATTN_F32(5); break;
    case 6: LC_ATTN_F32(6); break;
    case 7: LC_ATTN_F32(7); break;
    default: LC_ATTN_F32(8); break;
  }
#undef LC_ATTN_F32
  return hipGetLastError();
}

hipError_t attentionHalf(const uint16_t* q, const uint16_t* k, const uint16_t* vt, float* out_f32,
                         uint16_t* out_heads_concat, int heads, int bh, int S, int S_pad, int D, bool causal, Half t,
                         hipStream_t stream) {
  if (S <= 0 || bh <= 0 || S_pad % 128 != 0 || S_pad < S || (D != 64 && D != 128)) {
    return hipErrorInvalidValue;
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(D));
  const dim3 grid(bh, S_pad / 128);
  const int cz = causal ? 1 : 0;
  if (t == Half::kBF16) {
    if (D == 64) {
      hipLaunchKernelGGL((attn_fwd_half_kernel<BF16, 64>), grid, dim3(256), 0, stream, q, k, vt, out_f32,
                         out_heads_concat, heads, S, S_pad, cz, scale);
    } else {
      hipLaunchKernelGGL((attn_fwd_half_kernel<BF16, 128>), grid, dim3(256), 0, stream, q, k, vt, out_f32,
                         out_heads_concat, heads, S, S_pad, cz, scale);
    }
  } else {
    if (D == 64) {
      hipLaunchKernelGGL((attn_fwd_half_kernel<F16, 64>), grid, dim3(256), 0, stream, q, k, vt, out_f32,
                         out_heads_concat, heads, S, S_pad, cz, scale);
    } else {
      hipLaunchKernelGGL((attn_fwd_half_kernel<F16, 128>), grid, dim3(256), 0, stream, q, k, vt, out_f32,
                         out_heads_concat, heads, S, S_pad, cz, scale);
    }
  }
  return hipGetLastError();
}

}  // namespace lchip::kern
