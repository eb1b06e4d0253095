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

#include <type_traits>

#include "../kernels.hpp"
#include "kcommon.hpp"

namespace lchip::k {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaskValue = -1e30f;

// ---------------------------------------------------------------------------
// fp32: KS waves per 32 queries, v_mfma_f32_32x32x2_f32, D padded to 32*DT
// (zeros).  Wave w of the workgroup takes the 32-key tiles j = w, w+KS, ...
// with its own K / V tiles in LDS and its own online-softmax state; the KS
// partial states are merged through LDS at the end (m = max m_w, O and l
// rescaled by exp2(m_w - m) and summed in wave order).  KS > 1 puts more
// waves on small problems (one head of S = 256 is 8 query blocks).
// ---------------------------------------------------------------------------
// Where the fp32 attention kernel reads Q, K and V (element i of the
// [BH, S, D] layout).  kLds: floats of LDS the source keeps; kVec: K and V
// rows are plain 16-byte aligned global memory (float4 prefetch allowed).
struct AttnSrcGlobal {
  const float* q;
  const float* k;
  const float* v;
  DoneFlag done{};
  static constexpr int kLds = 0;
  static constexpr bool kVec = true;
  static constexpr bool kClamp = false;  // padding cells are not loaded
  // A position is the flat element index; W selects Q (0), K (1) or V (2).
  using Pos = size_t;
  __device__ void prologue(float*, int) const {}
  template <int W>
  __device__ Pos at(size_t i) const { return i; }
  __device__ size_t delta(size_t d) const { return d; }
  __device__ Pos fwd(Pos p, size_t d) const { return p + d; }
  template <int W>
  __device__ float ld(const float*, Pos p) const { return (W == 0 ? q : W == 1 ? k : v)[p]; }
  __device__ bool single_writer() const { return done.single_writer(); }
  __device__ void finish() const { done.finish(); }
};

// The reference's conv -> attention chain (bind_integrated.cpp:614-730):
// conv2d NCHW + bias + ReLU, then Q, K, V = consecutive S*D slices of the
// flat conv output, tiled by repetition when it holds fewer than 3*S*D values
// (QkvPackRepeat, :709-729).  Each workgroup computes the whole conv output
// (n <= kOut values) into LDS once, accumulating over (c, ky, kx) in im2col
// column order and adding the bias last as the reference's GEMM + scatter
// does; Q / K / V are then read from it by index.
struct AttnSrcConvRepeat {
  const float* x;
  const float* w;
  const float* bias;
  int cin, h, wd, cout, kh, kw, sh, sw, ph, pw, oh, ow;
  int n;        // conv output values (batch * cout * oh * ow), at most kOut
  int xs, ws;   // input and weight values
  size_t need;  // S * D
  DoneFlag done{};  // optional completion flag
  static constexpr int kOut = 8192;
  static constexpr int kLds = 12288;
  static constexpr bool kVec = false;
  static constexpr bool kClamp = true;  // every position is in bounds: padding loads a real value
  // Positions are indices into the conv output (< n): element i of Q, K, V
  // is conv[(W * S * D + i) mod n].  A fill walks its tile with pre-reduced
  // strides (one conditional subtract per step instead of a division).
  using Pos = uint32_t;
  __device__ void prologue(float* buf, int nthreads) const {
    // x, w and bias are staged behind the output when they fit (one
    // coalesced pass, then LDS reads instead of dependent global loads per
    // multiply-add).
    if (staged()) {
      // x, w and bias land back to back behind the output; one loop issues
      // all of their loads before any wait, so a source in mapped host
      // memory costs one PCIe round trip per workgroup instead of three.
      float* xb = buf + n;
      const int nb = bias != nullptr ? cout : 0;
      const int tot = xs + ws + nb;
      for (int i = threadIdx.x; i < tot; i += nthreads) {
        xb[i] = i < xs ? x[i] : (i < xs + ws ? w[i - xs] : bias[i - xs - ws]);
      }
      __syncthreads();
      conv(buf, xb, xb + xs, nb != 0 ? xb + xs + ws : nullptr, nthreads);
    } else {
      conv(buf, x, w, bias, nthreads);
    }
    __syncthreads();
  }
  // x, w and bias all fit in LDS next to the output: the only case in which
  // they are read from global memory once per workgroup (the host may then
  // hand over mapped host memory).
  __host__ __device__ bool staged() const { return n + xs + ws + cout <= kLds; }
  __device__ void conv(float* buf, const float* xp, const float* wp, const float* bp, int nthreads) const {
    const int hw = oh * ow;
    if (kh == 3 && kw == 3 && cin <= 4) {
      conv3x3(buf, xp, wp, bp, nthreads);
      return;
    }
    for (int f = threadIdx.x; f < n; f += nthreads) {
      const int t = f / hw;
      const int pix = f - t * hw;
      const int oy = pix / ow;
      const int ox = pix - oy * ow;
      const int oc = t % cout;
      const int b = t / cout;
      float acc = 0.0f;
      for (int c = 0; c < cin; ++c) {
        const float* xc = xp + (static_cast<size_t>(b) * cin + c) * h * wd;
        const float* wc = wp + (static_cast<size_t>(oc) * cin + c) * kh * kw;
        for (int ky = 0; ky < kh; ++ky) {
          const int iy = oy * sh + ky - ph;
          for (int kx = 0; kx < kw; ++kx) {
            const int ix = ox * sw + kx - pw;
            const float xv = (iy >= 0 && iy < h && ix >= 0 && ix < wd) ? xc[iy * wd + ix] : 0.0f;
            acc += xv * wc[ky * kw + kx];
          }
        }
      }
      if (bp != nullptr) {
        acc += bp[oc];
      }
      buf[f] = acc > 0.0f ? acc : 0.0f;
    }
  }
  // 3x3 kernels with at most 4 input channels (the hotspot shapes): one
  // thread per (output pixel, group of output channels).  The pixel's cin*9
  // inputs are loaded once (clamped in-bounds loads, zeroed outside the
  // image) and reused for every channel of the group; a wave's pixels share
  // their channel, so each weight read is one LDS broadcast.  Same
  // accumulation order as the general loop: (c, ky, kx), bias last.
  __device__ void conv3x3(float* buf, const float* xp, const float* wp, const float* bp, int nthreads) const {
    const int hw = oh * ow;
    const int npix = n / cout;  // batch * oh * ow
    int groups = nthreads / npix;
    groups = groups < 1 ? 1 : (groups > cout ? cout : groups);
    const int ocb = (cout + groups - 1) / groups;
    for (int item = threadIdx.x; item < npix * groups; item += nthreads) {
      const int g = item / npix;
      const int pix = item - g * npix;
      const int b = pix / hw;
      const int rem = pix - b * hw;
      const int oy = rem / ow;
      const int ox = rem - oy * ow;
      float xv[36];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (c < cin) {
          const float* xc = xp + (static_cast<size_t>(b) * cin + c) * h * wd;
#pragma unroll
          for (int ky = 0; ky < 3; ++ky) {
            const int iy = oy * sh + ky - ph;
            const int iyc = min(max(iy, 0), h - 1);
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
              const int ix = ox * sw + kx - pw;
              const int ixc = min(max(ix, 0), wd - 1);
              const float v = xc[iyc * wd + ixc];
              xv[c * 9 + ky * 3 + kx] = (iy == iyc && ix == ixc) ? v : 0.0f;
            }
          }
        }
      }
      const int oc_end = min(cout, (g + 1) * ocb);
      float* dst = buf + static_cast<size_t>(b) * cout * hw + rem;
      for (int oc = g * ocb; oc < oc_end; ++oc) {
        const float* wc = wp + oc * cin * 9;
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (c < cin) {
#pragma unroll
            for (int e = 0; e < 9; ++e) {
              acc += xv[c * 9 + e] * wc[c * 9 + e];
            }
          }
        }
        if (bp != nullptr) {
          acc += bp[oc];
        }
        dst[oc * hw] = acc > 0.0f ? acc : 0.0f;
      }
    }
  }
  // 32-bit index arithmetic (the host keeps 3*S*D below 2^31).
  template <int W>
  __device__ Pos at(size_t i) const {
    return static_cast<uint32_t>(W * need + i) % static_cast<uint32_t>(n);
  }
  __device__ uint32_t delta(size_t d) const { return static_cast<uint32_t>(d % static_cast<size_t>(n)); }
  __device__ Pos fwd(Pos p, uint32_t d) const {
    p += d;
    return p >= static_cast<uint32_t>(n) ? p - static_cast<uint32_t>(n) : p;
  }
  template <int W>
  __device__ float ld(const float* buf, Pos p) const { return buf[p]; }
  __device__ bool single_writer() const { return done.single_writer(); }
  __device__ void finish() const { done.finish(); }
};

// Fills rows row0, row0 + rstep, ... (< ROWS) of ROWS x DP tiles (row stride
// ldd) with operands W0 (and W1 when NT = 2) of rows first + r of one head;
// rows >= S and columns >= D are zero.  Lane l covers column l (and l + 64,
// ...) of a row, or for DP < 64 a column of one of 64 / DP adjacent rows
// (DP = 48: lanes 48-63 repeat columns 0-15 of the next row, the same value).
// The operands share positions: their loads are issued together.
template <int DP, int NT, int W0, int W1, typename Src, int ROWS = 32>
__device__ inline void fill_rows(const Src& src, const float* buf, float* dst0, int ldd0, float* dst1, int ldd1,
                                 int row0, int rstep, int first, int S, int D, size_t head, int lane) {
  constexpr int RPI = DP >= 64 ? 1 : 64 / DP;
  constexpr int CPR = DP >= 64 ? (DP + 63) / 64 : 1;
  const int lr = DP >= 64 ? 0 : lane / DP;
  const int lc = DP >= 64 ? lane : lane % DP;
  const int rstride = rstep * RPI;
  const int r0 = row0 * RPI + lr;
  const size_t flat = head + static_cast<size_t>(first + r0) * D + lc;
  auto p0 = src.template at<W0>(flat);
  auto p1 = src.template at<W1>(flat);
  // kClamp: padding cells load element 0 of the head (always in bounds) and
  // store zero, so every load is unconditional and the unrolled rows' loads
  // overlap instead of each sitting in its own exec-masked block.
  const auto z0 = src.template at<W0>(head);
  const auto z1 = src.template at<W1>(head);
  const auto drow = src.delta(static_cast<size_t>(rstride) * D);
  decltype(src.delta(0)) dch[CPR];
#pragma unroll
  for (int ch = 0; ch < CPR; ++ch) {
    dch[ch] = src.delta(static_cast<size_t>(64 * ch));
  }
#pragma unroll 8
  for (int r = r0; r < ROWS; r += rstride) {
    const bool rok = first + r < S;
#pragma unroll
    for (int ch = 0; ch < CPR; ++ch) {
      const int c = lc + 64 * ch;
      if (c < DP) {
        const bool ok = rok && c < D;
        if constexpr (Src::kClamp) {
          const float v0 = src.template ld<W0>(buf, ok ? (ch == 0 ? p0 : src.fwd(p0, dch[ch])) : z0);
          dst0[r * ldd0 + c] = ok ? v0 : 0.0f;
          if constexpr (NT == 2) {
            const float v1 = src.template ld<W1>(buf, ok ? (ch == 0 ? p1 : src.fwd(p1, dch[ch])) : z1);
            dst1[r * ldd1 + c] = ok ? v1 : 0.0f;
          }
        } else {
          dst0[r * ldd0 + c] = ok ? src.template ld<W0>(buf, ch == 0 ? p0 : src.fwd(p0, dch[ch])) : 0.0f;
          if constexpr (NT == 2) {
            dst1[r * ldd1 + c] = ok ? src.template ld<W1>(buf, ch == 0 ? p1 : src.fwd(p1, dch[ch])) : 0.0f;
          }
        }
      }
    }
    p0 = src.fwd(p0, drow);
    if constexpr (NT == 2) {
      p1 = src.fwd(p1, drow);
    }
  }
}

template <int DT, int KS, bool VEC, typename Src>
__global__ __launch_bounds__(64 * KS) void attn_fwd_f32_kernel(Src src, float* __restrict__ out,
                                                               float* __restrict__ stats, int S, int D, int causal,
                                                               float scale, float post_scale, float post_bias,
                                                               int post_relu, int split_tiles, float* __restrict__ ws) {
  constexpr int DP = 32 * DT;
  // Q and K rows have stride DP + 4: 16-byte aligned (float4 reads), and a
  // 16-lane pass of one float4 per row touches 16 distinct bank groups.
  constexpr int QKS = DP + 4;
  constexpr int KV = 32 * QKS + 32 * DP;  // floats of one wave's K + V tile
  static_assert(!VEC || Src::kVec, "vector prefetch needs a global source");
  __shared__ __attribute__((aligned(16))) float Qs[32][QKS];
  __shared__ __attribute__((aligned(16))) float kv[KS][KV];
  __shared__ float srcbuf[Src::kLds > 0 ? Src::kLds : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float (*Ks)[QKS] = reinterpret_cast<float (*)[QKS]>(&kv[wave][0]);
  float (*Vs)[DP] = reinterpret_cast<float (*)[DP]>(&kv[wave][32 * QKS]);
  // Workgroup qb: query block qb; its waves take the 32-key tiles w + KS n.
  // Heaviest (causal) blocks first.  Key split (split_tiles > 0): workgroup
  // z = blockIdx.z takes only the tiles [z, z + 1) * split_tiles and writes
  // its unnormalised partial (O, m, l) to ws for attn_split_combine_kernel:
  // O [z][head][S][D], then (m, l) [z][head][S][2].
  const bool split = split_tiles > 0;
  const int nqb = (S + 31) / 32;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x);
  const int q0 = qb * 32;
  const int kbeg = split ? static_cast<int>(blockIdx.z) * split_tiles * 32 : 0;
  const int jfirst = kbeg + wave * 32;
  const int jstep = 32 * KS;
  const size_t head = static_cast<size_t>(blockIdx.y) * S * D;
  float* ml = nullptr;
  if (split) {
    out = ws + static_cast<size_t>(blockIdx.z) * gridDim.y * S * D;
    ml = ws + static_cast<size_t>(gridDim.z) * gridDim.y * S * D +
         (static_cast<size_t>(blockIdx.z) * gridDim.y + blockIdx.y) * S * 2;
  }
  out += head;
  src.prologue(srcbuf, 64 * KS);

  floatx16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    o[t] = zero16();
  }
  float m_run = kMaskValue;
  float l_run = 0.0f;
  const int qi = q0 + (lane & 31);
  int kend = causal ? min(S, q0 + 32) : S;
  if (split) {
    kend = min(kend, kbeg + split_tiles * 32);
  }

  // Only this wave touches its K / V tiles: wave-level ordering suffices
  // (LDS accesses of one wave complete in order).  VEC (D % 4 == 0, 16-byte
  // aligned rows): tiles move as float4.  DT <= 2 (PREF): each lane holds CH
  // float4 of the next tile's K and V in registers, loaded while the current
  // tile is computed; wider tiles (FILL4) are loaded and stored in groups of
  // four chunks at the top of each tile.
  constexpr bool PREF = VEC && DT <= 2;
  constexpr bool FILL4 = VEC && DT > 2;
  constexpr int CH = DP / 8;  // float4 chunks per lane per operand
  float4 kr[PREF ? CH : 1];
  float4 vr[PREF ? CH : 1];
  auto fetch = [&](int j0) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int idx = c * 64 + lane;  // chunk: row idx / (DP/4), column 4 * (idx % (DP/4))
      const int r = idx / (DP / 4);
      const int cc = (idx - r * (DP / 4)) * 4;
      const bool ok = j0 + r < S && cc < D;
      const size_t off = static_cast<size_t>(j0 + r) * D + cc;
      if constexpr (PREF) {
        kr[c] = ok ? *reinterpret_cast<const float4*>(src.k + head + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        vr[c] = ok ? *reinterpret_cast<const float4*>(src.v + head + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  };
  // The first K / V tile's loads go out before the Q tile's, so their
  // latencies overlap.
  if constexpr (PREF) {
    if (jfirst < kend) {
      fetch(jfirst);
    }
  }
  fill_rows<DP, 1, 0, 0>(src, srcbuf, &Qs[0][0], QKS, nullptr, 0, wave, KS, q0, S, D, head, lane);
  __syncthreads();
  for (int j0 = jfirst; j0 < kend; j0 += jstep) {
    if constexpr (PREF) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int idx = c * 64 + lane;
        const int r = idx / (DP / 4);
        const int cc = (idx - r * (DP / 4)) * 4;
        *reinterpret_cast<float4*>(&Ks[r][cc]) = kr[c];
        *reinterpret_cast<float4*>(&Vs[r][cc]) = vr[c];
      }
      if (j0 + jstep < kend) {
        fetch(j0 + jstep);
      }
    } else if constexpr (FILL4) {
      for (int c0 = 0; c0 < CH; c0 += 4) {
        float4 kx[4];
        float4 vx[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int idx = (c0 + c) * 64 + lane;
          const int r = idx / (DP / 4);
          const int cc = (idx - r * (DP / 4)) * 4;
          const bool ok = j0 + r < S && cc < D;
          const size_t off = static_cast<size_t>(j0 + r) * D + cc;
          kx[c] = ok ? *reinterpret_cast<const float4*>(src.k + head + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          vx[c] = ok ? *reinterpret_cast<const float4*>(src.v + head + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int idx = (c0 + c) * 64 + lane;
          const int r = idx / (DP / 4);
          const int cc = (idx - r * (DP / 4)) * 4;
          *reinterpret_cast<float4*>(&Ks[r][cc]) = kx[c];
          *reinterpret_cast<float4*>(&Vs[r][cc]) = vx[c];
        }
      }
    } else {
      fill_rows<DP, 2, 1, 2>(src, srcbuf, &Ks[0][0], QKS, &Vs[0][0], DP, 0, 1, j0, S, D, head, lane);
    }
    __builtin_amdgcn_wave_barrier();

    // Over the padded DP (columns D..DP-1 of both tiles are zero).  The k
    // order inside the MFMAs is free as long as K and Q agree: lane half h
    // takes k in [h DP/2, (h+1) DP/2), so each lane reads 4 k at a time.
    floatx16 st = zero16();
    {
      const float* krow = &Ks[lane & 31][(lane >> 5) * (DP / 2)];
      const float* qrow = &Qs[lane & 31][(lane >> 5) * (DP / 2)];
#pragma unroll
      for (int k4 = 0; k4 < DP / 2; k4 += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(krow + k4);
        const float4 b4 = *reinterpret_cast<const float4*>(qrow + k4);
        st = mfma32x32x2f32(a4.x, b4.x, st);
        st = mfma32x32x2f32(a4.y, b4.y, st);
        st = mfma32x32x2f32(a4.z, b4.z, st);
        st = mfma32x32x2f32(a4.w, b4.w, st);
      }
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
    __builtin_amdgcn_wave_barrier();  // the next tile overwrites K / V of this one
  }

  l_run += __shfl_xor(l_run, 32);
  // The normalised 32 x D output block is assembled in Qs' storage (free:
  // every wave is past its QK^T) with row stride DP + 1, so writes by query
  // are free of bank conflicts, and then stored as contiguous rows by every
  // wave: full lines in HBM, and few large transactions when out is mapped
  // host memory.
  constexpr int TS = DP + 1;
  float* tile = &Qs[0][0];
  auto post = [&](float val) {
    if (post_scale != 1.0f || post_bias != 0.0f || post_relu) {
      val = val * post_scale + post_bias;
      if (post_relu && val < 0.0f) {
        val = 0.0f;
      }
    }
    return val;
  };
  const int ql = lane & 31;
  if (KS > 1) {
    // Park each wave's state in its own K / V region: m, l (32 each), then
    // O^T as [query][d] (row stride DP + 1).  A wave that saw no key tile
    // parks m = -1e30, l = 0.
    constexpr int PS = DP + 1;
    float* mine = &kv[wave][0];
    if (lane < 32) {
      mine[lane] = m_run;
      mine[32 + lane] = l_run;
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        mine[64 + ql * PS + t * 32 + acc_row(i, lane)] = o[t][i];
      }
    }
    __syncthreads();
    // Every wave merges a share: lane (ql, half) of wave w takes the output
    // columns d = 2 (w + KS n) + half of query ql.
    float m_all = kMaskValue;
#pragma unroll
    for (int w = 0; w < KS; ++w) {
      m_all = fmaxf(m_all, kv[w][ql]);
    }
    float f[KS];
    float l_all = 0.0f;
#pragma unroll
    for (int w = 0; w < KS; ++w) {
      f[w] = exp2f(kv[w][ql] - m_all);
      l_all += f[w] * kv[w][32 + ql];
    }
    const float inv = 1.0f / l_all;
    // Row statistics for a later pass that recomputes P (the train
    // step's dV): p = exp2(x - m) / l with x = (q.k) * scale * log2(e).
    if (stats != nullptr && wave == 0 && lane < 32 && qi < S) {
      stats[(static_cast<size_t>(blockIdx.y) * S + qi) * 2] = m_all;
      stats[(static_cast<size_t>(blockIdx.y) * S + qi) * 2 + 1] = l_all;
    }
    if (split && wave == 0 && lane < 32 && qi < S) {
      ml[qi * 2] = m_all;
      ml[qi * 2 + 1] = l_all;
    }
    for (int d = 2 * wave + (lane >> 5); d < D; d += 2 * KS) {
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < KS; ++w) {
        acc += f[w] * kv[w][64 + ql * PS + d];
      }
      tile[ql * TS + d] = split ? acc : post(acc * inv);
    }
  } else {
    const float inv = 1.0f / l_run;
    if (stats != nullptr && lane < 32 && qi < S) {
      stats[(static_cast<size_t>(blockIdx.y) * S + qi) * 2] = m_run;
      stats[(static_cast<size_t>(blockIdx.y) * S + qi) * 2 + 1] = l_run;
    }
    if (split && lane < 32 && qi < S) {
      ml[qi * 2] = m_run;
      ml[qi * 2 + 1] = l_run;
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = t * 32 + acc_row(i, lane);
        if (d < D) {
          tile[ql * TS + d] = split ? o[t][i] : post(o[t][i] * inv);
        }
      }
    }
  }
  __syncthreads();
  // Rows q0 .. q0 + rows - 1 are one contiguous range of out; wave w stores
  // rows w, w + KS, ..., its lanes over the columns.
  const int rows = min(32, S - q0);
  float* dst = out + static_cast<size_t>(q0) * D;
  const bool one = src.single_writer();
  if (!one || wave == 0) {
    for (int r = one ? 0 : wave; r < rows; r += one ? 1 : KS) {
#pragma unroll
      for (int c0 = 0; c0 < DP; c0 += 64) {
        const int c = c0 + lane;
        if (c < D) {
          dst[r * D + c] = tile[r * TS + c];
        }
      }
    }
  }
  src.finish();
}

// Merges attn_fwd_f32_kernel's key splits: per query row, M = max_z m_z,
// L = sum_z l_z exp2(m_z - M) and out = post(sum_z O_z exp2(m_z - M) / L),
// splits summed in z order; stats (optional) receive (M, L).  One wave per
// row, four rows per workgroup; every thread reaches the completion flag.
__global__ __launch_bounds__(256) void attn_split_combine_kernel(const float* __restrict__ ws, float* __restrict__ out,
                                                                 float* __restrict__ stats, int rows, int D,
                                                                 int nsplit, float post_scale, float post_bias,
                                                                 int post_relu, DoneFlag done) {
  const int row = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row < rows) {
    const float* ml = ws + static_cast<size_t>(nsplit) * rows * D;
    float m_all = kMaskValue;
    for (int z = 0; z < nsplit; ++z) {
      m_all = fmaxf(m_all, ml[(static_cast<size_t>(z) * rows + row) * 2]);
    }
    float l_all = 0.0f;
    for (int z = 0; z < nsplit; ++z) {
      const float* p = ml + (static_cast<size_t>(z) * rows + row) * 2;
      l_all += p[1] * exp2f(p[0] - m_all);
    }
    const float inv = 1.0f / l_all;
    for (int d = lane; d < D; d += 64) {
      float acc = 0.0f;
      for (int z = 0; z < nsplit; ++z) {
        acc += ws[(static_cast<size_t>(z) * rows + row) * D + d] *
               exp2f(ml[(static_cast<size_t>(z) * rows + row) * 2] - m_all);
      }
      float val = acc * inv;
      if (post_scale != 1.0f || post_bias != 0.0f || post_relu) {
        val = val * post_scale + post_bias;
        if (post_relu && val < 0.0f) {
          val = 0.0f;
        }
      }
      out[static_cast<size_t>(row) * D + d] = val;
    }
    if (stats != nullptr && lane == 0) {
      stats[static_cast<size_t>(row) * 2] = m_all;
      stats[static_cast<size_t>(row) * 2 + 1] = l_all;
    }
  }
  done.finish_all_writers();
}

// ---------------------------------------------------------------------------
// fp32 attention for problems too small to fill the GPU (one head, S of a few
// hundred): 16 queries per workgroup and KS waves (8 up to S = 256, else
// 16), wave w taking the 16-key tiles w, w + KS, ... with
// v_mfma_f32_16x16x4_f32.  At S = 256 that is 16 workgroups x 8 waves, each
// wave two 16 x 16 score tiles (16 + 16 MFMAs of 32 cycles each) where
// attn_fwd_f32_kernel<2, 8> gives each of its 64 waves a 32 x 32 tile (64
// MFMAs of 64 cycles).  D <= 64, D % 4 == 0 and
// 16-byte aligned K / V rows (float4 loads); the KS states merge through LDS
// as in attn_fwd_f32_kernel.
//
// Scores are S^T = K . Q^T per tile: lane l holds keys 4g + i (g = l / 16,
// i = 0..3) of query c = l % 16.  The QK^T reduction over d gives lane group
// g the d range [g DP/4, (g+1) DP/4).  For O^T += V^T . P^T, k-step s takes
// keys {4g + s}, so each lane feeds its own probability st[s] as the B operand
// and reads V row 4g + s; output row d = 16 dt + 4g + i, column c.
// ---------------------------------------------------------------------------
template <int DQ, int KS, typename Src>
__global__ __launch_bounds__(64 * KS) void attn_fwd_f32_q16_kernel(Src src, float* __restrict__ out,
                                                                   float* __restrict__ stats, int S, int D,
                                                                   int causal, float scale, float post_scale,
                                                                   float post_bias, int post_relu) {
  constexpr int DP = 16 * DQ;
  constexpr int QS = DP + 4;             // Q / K row stride (16-byte aligned rows)
  constexpr int KVF = 16 * QS + 16 * DP; // floats of one wave's K + V tile
  constexpr int PS = DP + 1;             // parked O row stride
  static_assert(DQ >= 1 && DQ <= 4 && 32 + 16 * PS <= KVF, "tile");
  __shared__ __attribute__((aligned(16))) float Qs[16 * QS];
  __shared__ __attribute__((aligned(16))) float kv[KS][KVF];
  __shared__ float srcbuf[Src::kLds > 0 ? Src::kLds : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  float* Ks = &kv[wave][0];
  float* Vs = &kv[wave][16 * QS];
  const int nqb = (S + 15) / 16;
  const int q0 = (nqb - 1 - static_cast<int>(blockIdx.x)) * 16;  // heaviest (causal) blocks first
  const size_t head = static_cast<size_t>(blockIdx.y) * S * D;
  const int qi = q0 + c;
  const int kend = causal ? min(S, q0 + 16) : S;
  const int jfirst = wave * 16;
  constexpr int jstep = 16 * KS;
  src.prologue(srcbuf, 64 * KS);

  // Global sources (Src::kVec): one tile of K and V is 16 rows x DP/4
  // float4, DQ chunks per lane each, prefetched one tile ahead in registers.
  // Other sources fill the tiles through the source's positions.
  constexpr bool VEC = Src::kVec;
  float4 kr[VEC ? DQ : 1], vr[VEC ? DQ : 1];
  auto fetch = [&](int j0) {
    if constexpr (VEC) {
#pragma unroll
      for (int t = 0; t < DQ; ++t) {
        const int idx = t * 64 + lane;  // row idx / (DP/4), column 4 (idx % (DP/4))
        const int r = idx / (DP / 4);
        const int cc = (idx - r * (DP / 4)) * 4;
        const bool ok = j0 + r < S && cc < D;
        const size_t off = head + static_cast<size_t>(j0 + r) * D + cc;
        kr[t] = ok ? *reinterpret_cast<const float4*>(src.k + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        vr[t] = ok ? *reinterpret_cast<const float4*>(src.v + off) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  };
  if constexpr (VEC) {
    if (jfirst < kend) {
      fetch(jfirst);  // out before the Q loads, so the latencies overlap
    }
    for (int idx = threadIdx.x; idx < 16 * (DP / 4); idx += 64 * KS) {
      const int r = idx / (DP / 4);
      const int cc = (idx - r * (DP / 4)) * 4;
      const bool ok = q0 + r < S && cc < D;
      *reinterpret_cast<float4*>(&Qs[r * QS + cc]) =
          ok ? *reinterpret_cast<const float4*>(src.q + head + static_cast<size_t>(q0 + r) * D + cc)
             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  } else {
    fill_rows<DP, 1, 0, 0, Src, 16>(src, srcbuf, Qs, QS, nullptr, 0, wave, KS, q0, S, D, head, lane);
  }
  __syncthreads();

  floatx4 o[DQ];
#pragma unroll
  for (int t = 0; t < DQ; ++t) {
    o[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  float m_run = kMaskValue;
  float l_run = 0.0f;
  for (int j0 = jfirst; j0 < kend; j0 += jstep) {
    if constexpr (VEC) {
#pragma unroll
      for (int t = 0; t < DQ; ++t) {
        const int idx = t * 64 + lane;
        const int r = idx / (DP / 4);
        const int cc = (idx - r * (DP / 4)) * 4;
        *reinterpret_cast<float4*>(&Ks[r * QS + cc]) = kr[t];
        *reinterpret_cast<float4*>(&Vs[r * DP + cc]) = vr[t];
      }
      if (j0 + jstep < kend) {
        fetch(j0 + jstep);
      }
    } else {
      fill_rows<DP, 2, 1, 2, Src, 16>(src, srcbuf, Ks, QS, Vs, DP, 0, 1, j0, S, D, head, lane);
    }
    __builtin_amdgcn_wave_barrier();  // only this wave reads its K / V tile

    floatx4 st = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    {
      const float* krow = &Ks[c * QS + g * (DP / 4)];
      const float* qrow = &Qs[c * QS + g * (DP / 4)];
#pragma unroll
      for (int t4 = 0; t4 < DP / 4; t4 += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(krow + t4);
        const float4 b4 = *reinterpret_cast<const float4*>(qrow + t4);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, b4.x, st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, b4.y, st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, b4.z, st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, b4.w, st, 0, 0, 0);
      }
    }
    float mt = kMaskValue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = j0 + 4 * g + i;
      // (q.k) * scale as the reference, then to the log2 domain
      float x = (st[i] * scale) * kLog2e;
      if (key >= S || (causal && key > qi)) {
        x = kMaskValue;
      }
      st[i] = x;
      mt = fmaxf(mt, x);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = exp2f(m_run - m_new);
    float ls = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = exp2f(st[i] - m_new);
      st[i] = p;
      ls += p;
    }
    l_run = l_run * alpha + ls;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < DQ; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[t][i] *= alpha;
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int t = 0; t < DQ; ++t) {
        const float a = Vs[(4 * g + s) * DP + t * 16 + c];
        o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, st[s], o[t], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next tile overwrites K / V of this one
  }
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);

  // Park each wave's state in its K / V region: m, l (16 each), then O as
  // [query][d] (row stride DP + 1); a wave that saw no tile parks m = -1e30,
  // l = 0, O = 0.
  float* mine = &kv[wave][0];
  if (lane < 16) {
    mine[lane] = m_run;
    mine[16 + lane] = l_run;
  }
#pragma unroll
  for (int t = 0; t < DQ; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mine[32 + c * PS + t * 16 + 4 * g + i] = o[t][i];
    }
  }
  __syncthreads();
  // The merge factors exp2(m_w - m_all), once per (query, wave) pair, into
  // the unused tail of wave 0's region (past its parked O).
  constexpr int FOFF = (32 + 16 * PS + 3) & ~3;
  static_assert(FOFF + 16 * (KS + 1) <= KVF, "merge factors fit");
  float* fw = &kv[0][FOFF];
  if (threadIdx.x < 16 * KS) {
    const int q = threadIdx.x & 15;
    const int w = threadIdx.x >> 4;
    float mq = kMaskValue;
#pragma unroll
    for (int u = 0; u < KS; ++u) {
      mq = fmaxf(mq, kv[u][q]);
    }
    fw[16 + w * 16 + q] = exp2f(kv[w][q] - mq);
    if (w == 0) {
      fw[q] = mq;
    }
  }
  __syncthreads();
  // Thread (query ql, slot) merges output columns d = slot, slot + 4 KS, ...
  const int ql = threadIdx.x & 15;
  const int slot = threadIdx.x >> 4;
  const float m_all = fw[ql];
  float f[KS];
  float l_all = 0.0f;
#pragma unroll
  for (int w = 0; w < KS; ++w) {
    f[w] = fw[16 + w * 16 + ql];
    l_all += f[w] * kv[w][16 + ql];
  }
  const float inv = 1.0f / l_all;
  // Row statistics for a pass that recomputes P (the train step's dV):
  // p = exp2(x - m) / l with x = (q.k) * scale * log2(e).
  if (stats != nullptr && threadIdx.x < 16 && q0 + ql < S) {
    stats[(static_cast<size_t>(blockIdx.y) * S + q0 + ql) * 2] = m_all;
    stats[(static_cast<size_t>(blockIdx.y) * S + q0 + ql) * 2 + 1] = l_all;
  }
  constexpr int TS = DP + 1;
  float* tile = Qs;  // 16 x (DP + 1) <= 16 x QS floats; every wave is past its QK^T
  for (int d = slot; d < D; d += 4 * KS) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < KS; ++w) {
      acc += f[w] * kv[w][32 + ql * PS + d];
    }
    float val = acc * inv;
    if (post_scale != 1.0f || post_bias != 0.0f || post_relu) {
      val = val * post_scale + post_bias;
      if (post_relu && val < 0.0f) {
        val = 0.0f;
      }
    }
    tile[ql * TS + d] = val;
  }
  __syncthreads();
  // Rows q0 .. q0 + rows - 1 are one contiguous range of out.
  const int rows = min(16, S - q0);
  float* dst = out + head + static_cast<size_t>(q0) * D;
  const bool one = src.single_writer();
  if (!one || wave == 0) {
    for (int r = one ? 0 : wave; r < rows; r += one ? 1 : KS) {
      if (lane < D) {
        dst[r * D + lane] = tile[r * TS + lane];
      }
    }
  }
  src.finish();
}

// ---------------------------------------------------------------------------
// Train step backward (fp32): dV = P^T . dO with dO = 2 (out - target) / (S*D),
// then V -= lr * dV in place (the reference's attentionTrainStepCpu,
// src/attention_cpu.cpp:114-163).  P is not stored: the forward left each
// query's softmax statistics (m, l), and P[i][j] = exp2(x_ij - m_i) / l_i is
// recomputed tile by tile from the same x_ij = (q_i.k_j) * scale * log2(e).
//
// One workgroup per 32-key block, KS waves splitting its query tiles.  Scores
// are computed untransposed here, S = Q . K^T, so lane l holds key l % 32 and
// 16 queries; then dV^T += dO^T . P takes P straight from those registers as
// the B operand (query order acc_row(s, l) inside each k pair, the same
// permutation on dO^T).  The KS partial dV^T tiles are summed through LDS in
// wave order and applied by wave 0.
// ---------------------------------------------------------------------------
template <int DT, int KS>
__global__ __launch_bounds__(64 * KS) void attn_dv_f32_kernel(const float* __restrict__ q,
                                                              const float* __restrict__ k, float* __restrict__ v,
                                                              const float* __restrict__ out,
                                                              const float* __restrict__ target,
                                                              const float* __restrict__ stats, int S, int D,
                                                              int causal, float scale, float lr, int split_qt,
                                                              float* __restrict__ ws) {
  constexpr int DP = 32 * DT;
  constexpr int QO = 32 * (DP + 1) + 32 * DP;  // floats of one wave's Q + dO tile
  __shared__ float Ks[32][DP + 1];
  __shared__ __attribute__((aligned(16))) float qo[KS][QO];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float (*Qs)[DP + 1] = reinterpret_cast<float (*)[DP + 1]>(&qo[wave][0]);
  float (*Gs)[DP] = reinterpret_cast<float (*)[DP]>(&qo[wave][32 * (DP + 1)]);
  const int j0 = blockIdx.x * 32;  // first key of this block
  const size_t head = static_cast<size_t>(blockIdx.y) * S * D;
  q += head;
  k += head;
  v += head;
  out += head;
  target += head;
  stats += static_cast<size_t>(blockIdx.y) * S * 2;
  const float norm = 1.0f / (static_cast<float>(S) * static_cast<float>(D));

  for (int idx = threadIdx.x; idx < 32 * DP; idx += 64 * KS) {
    const int r = idx / DP;
    const int cc = idx - r * DP;
    Ks[r][cc] = (j0 + r < S && cc < D) ? k[static_cast<size_t>(j0 + r) * D + cc] : 0.0f;
  }
  __syncthreads();

  floatx16 dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    dv[t] = zero16();
  }
  const int key = j0 + (lane & 31);
  const int nqt = (S + 31) / 32;
  // Causal: query tile I meets key block J only when some query >= some key.
  // Query split (split_qt > 0): workgroup z = blockIdx.z takes only the query
  // tiles [z, z + 1) * split_qt and writes its partial dV [z][head][S][D] to
  // ws (zeros when it meets none); attn_dv_split_combine_kernel sums the
  // splits and updates V.
  const int qlo = split_qt > 0 ? static_cast<int>(blockIdx.z) * split_qt : 0;
  const int qhi = split_qt > 0 ? min(nqt, qlo + split_qt) : nqt;
  const bool vec = (D & 3) == 0;
  for (int qt = max(qlo, causal ? static_cast<int>(blockIdx.x) : 0) + wave; qt < qhi; qt += KS) {
    const int i0 = qt * 32;
    // This lane's 16 queries' softmax statistics, loaded first so their
    // latency overlaps the tile fills and QK^T.
    float sm[16];
    float sl[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = min(i0 + acc_row(r, lane), S - 1);
      sm[r] = stats[static_cast<size_t>(qi) * 2];
      sl[r] = stats[static_cast<size_t>(qi) * 2 + 1];
    }
    if (vec) {
      // float4 fills (D % 4 == 0: a chunk is all inside or all past D).
      for (int idx = lane; idx < 32 * (DP / 4); idx += 64) {
        const int r = idx / (DP / 4);
        const int cc = (idx - r * (DP / 4)) * 4;
        float4 qv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float4 gv = qv;
        if (i0 + r < S && cc < D) {
          const size_t off = static_cast<size_t>(i0 + r) * D + cc;
          qv = *reinterpret_cast<const float4*>(q + off);
          const float4 ov = *reinterpret_cast<const float4*>(out + off);
          const float4 tv = *reinterpret_cast<const float4*>(target + off);
          const float g = 2.0f * norm;
          gv = make_float4((ov.x - tv.x) * g, (ov.y - tv.y) * g, (ov.z - tv.z) * g, (ov.w - tv.w) * g);
        }
        Qs[r][cc] = qv.x;
        Qs[r][cc + 1] = qv.y;
        Qs[r][cc + 2] = qv.z;
        Qs[r][cc + 3] = qv.w;
        *reinterpret_cast<float4*>(&Gs[r][cc]) = gv;
      }
    } else {
      for (int idx = lane; idx < 32 * DP; idx += 64) {
        const int r = idx / DP;
        const int cc = idx - r * DP;
        const bool ok = i0 + r < S && cc < D;
        const size_t off = static_cast<size_t>(i0 + r) * D + cc;
        Qs[r][cc] = ok ? q[off] : 0.0f;
        Gs[r][cc] = ok ? 2.0f * (out[off] - target[off]) * norm : 0.0f;
      }
    }
    __builtin_amdgcn_wave_barrier();
    // S = Q . K^T: A = Q rows (query), B = K^T (lane: key, k = d).
    floatx16 st = zero16();
#pragma unroll
    for (int dd = 0; dd < DP; dd += 2) {
      const float a = Qs[lane & 31][dd + (lane >> 5)];
      const float b = Ks[lane & 31][dd + (lane >> 5)];
      st = mfma32x32x2f32(a, b, st);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = i0 + acc_row(r, lane);
      float p = 0.0f;
      if (qi < S && key < S && !(causal && key > qi)) {
        p = exp2f((st[r] * scale) * kLog2e - sm[r]) / sl[r];
      }
      st[r] = p;
    }
    // dV^T += dO^T . P: step r pairs queries acc_row(r, l) of both lane halves.
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = acc_row(r, lane);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const float a = Gs[qr][t * 32 + (lane & 31)];
        dv[t] = mfma32x32x2f32(a, st[r], dv[t]);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next query tile overwrites Q / dO
  }

  // Sum the KS partial dV^T tiles ([d][key]) and update V[key][d].
  if constexpr (KS > 1) {
    float* mine = &qo[wave][0];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        mine[(t * 32 + acc_row(r, lane)) * 32 + (lane & 31)] = dv[t][r];
      }
    }
    __syncthreads();
    if (wave != 0) {
      return;
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      // Four rows at a time: fully unrolled over 16 rows x KS waves, the
      // loads of KS = 8 push the kernel past its 256 registers into scratch.
#pragma unroll 4
      for (int r = 0; r < 16; ++r) {
        const int idx = (t * 32 + acc_row(r, lane)) * 32 + (lane & 31);
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < KS; ++w) {
          acc += qo[w][idx];
        }
        dv[t][r] = acc;
      }
    }
  }
  if (key < S) {
    float* part = split_qt > 0 ? ws + static_cast<size_t>(blockIdx.z) * gridDim.y * S * D + head : nullptr;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = t * 32 + acc_row(r, lane);
        if (d < D) {
          if (split_qt > 0) {
            part[static_cast<size_t>(key) * D + d] = dv[t][r];
          } else {
            float* vp = v + static_cast<size_t>(key) * D + d;
            *vp = *vp - lr * dv[t][r];
          }
        }
      }
    }
  }
}

// Sums attn_dv_f32_kernel's query splits in split order and applies
// V -= lr * dV, one thread per element of V.
__global__ __launch_bounds__(256) void attn_dv_split_combine_kernel(const float* __restrict__ ws, float* __restrict__ v,
                                                                    size_t n, int nsplit, float lr) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * 256) {
    float acc = 0.0f;
    for (int z = 0; z < nsplit; ++z) {
      acc += ws[static_cast<size_t>(z) * n + i];
    }
    v[i] = v[i] - lr * acc;
  }
}

// The train step's dV for small problems, the counterpart of
// attn_fwd_f32_q16_kernel: one workgroup per 16-key block and 16 waves taking
// its 16-query tiles w, w + KS, ... with v_mfma_f32_16x16x4_f32.  Scores are
// S = Q . K^T per tile, lane l holding queries 4g + i (g = l / 16) of key
// l % 16; dV^T += dO^T . P takes queries {4g + s} in k-step s, so each lane
// feeds its own probability as the B operand and reads dO row 4g + s.  The
// KS partial dV^T tiles are summed in wave order by all threads, each owning
// one (d, key) element, which then updates V.  D <= 64, D % 4 == 0, 16-byte
// aligned operands.
template <int DQ, int KS>
__global__ __launch_bounds__(64 * KS) void attn_dv_f32_q16_kernel(const float* __restrict__ q,
                                                                  const float* __restrict__ k, float* __restrict__ v,
                                                                  const float* __restrict__ out,
                                                                  const float* __restrict__ target,
                                                                  const float* __restrict__ stats, int S, int D,
                                                                  int causal, float scale, float lr) {
  constexpr int DP = 16 * DQ;
  constexpr int QS = DP + 4;              // Q / K row stride
  constexpr int QO = 16 * QS + 16 * DP;   // floats of one wave's Q + dO tile
  static_assert(DQ >= 1 && DQ <= 4 && 16 * DP <= QO, "tile");
  __shared__ __attribute__((aligned(16))) float Ks[16 * QS];
  __shared__ __attribute__((aligned(16))) float qo[KS][QO];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  float* Qs = &qo[wave][0];
  float* Gs = &qo[wave][16 * QS];
  const int j0 = blockIdx.x * 16;  // first key of this block
  const size_t head = static_cast<size_t>(blockIdx.y) * S * D;
  q += head;
  k += head;
  v += head;
  out += head;
  target += head;
  stats += static_cast<size_t>(blockIdx.y) * S * 2;
  const float g2 = 2.0f / (static_cast<float>(S) * static_cast<float>(D));

  for (int idx = threadIdx.x; idx < 16 * (DP / 4); idx += 64 * KS) {
    const int r = idx / (DP / 4);
    const int cc = (idx - r * (DP / 4)) * 4;
    *reinterpret_cast<float4*>(&Ks[r * QS + cc]) =
        (j0 + r < S && cc < D) ? *reinterpret_cast<const float4*>(k + static_cast<size_t>(j0 + r) * D + cc)
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  __syncthreads();

  floatx4 dv[DQ];
#pragma unroll
  for (int t = 0; t < DQ; ++t) {
    dv[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const int key = j0 + c;
  const int nqt = (S + 15) / 16;
  // Causal: query tile I meets key block J only when I >= J.
  for (int qt = (causal ? blockIdx.x : 0) + wave; qt < nqt; qt += KS) {
    const int i0 = qt * 16;
    // This lane's 4 queries' softmax statistics, loaded first so their
    // latency overlaps the tile fills and QK^T.
    float sm[4];
    float sl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qi = min(i0 + 4 * g + i, S - 1);
      sm[i] = stats[static_cast<size_t>(qi) * 2];
      sl[i] = stats[static_cast<size_t>(qi) * 2 + 1];
    }
#pragma unroll
    for (int t = 0; t < DQ; ++t) {
      const int idx = t * 64 + lane;
      const int r = idx / (DP / 4);
      const int cc = (idx - r * (DP / 4)) * 4;
      float4 qv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      float4 gv = qv;
      if (i0 + r < S && cc < D) {
        const size_t off = static_cast<size_t>(i0 + r) * D + cc;
        qv = *reinterpret_cast<const float4*>(q + off);
        const float4 ov = *reinterpret_cast<const float4*>(out + off);
        const float4 tv = *reinterpret_cast<const float4*>(target + off);
        gv = make_float4((ov.x - tv.x) * g2, (ov.y - tv.y) * g2, (ov.z - tv.z) * g2, (ov.w - tv.w) * g2);
      }
      *reinterpret_cast<float4*>(&Qs[r * QS + cc]) = qv;
      *reinterpret_cast<float4*>(&Gs[r * DP + cc]) = gv;
    }
    __builtin_amdgcn_wave_barrier();
    // S = Q . K^T: A = Q rows (query), B = K^T (key); lane group g reduces d
    // in [g DP/4, (g+1) DP/4).
    floatx4 st = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    {
      const float* qrow = &Qs[c * QS + g * (DP / 4)];
      const float* krow = &Ks[c * QS + g * (DP / 4)];
#pragma unroll
      for (int t4 = 0; t4 < DP / 4; t4 += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(qrow + t4);
        const float4 b4 = *reinterpret_cast<const float4*>(krow + t4);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, b4.x, st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, b4.y, st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, b4.z, st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, b4.w, st, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qi = i0 + 4 * g + i;
      float p = 0.0f;
      if (qi < S && key < S && !(causal && key > qi)) {
        p = exp2f((st[i] * scale) * kLog2e - sm[i]) / sl[i];
      }
      st[i] = p;
    }
    // dV^T += dO^T . P: k-step s takes queries {4g + s}.
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int t = 0; t < DQ; ++t) {
        const float a = Gs[(4 * g + s) * DP + t * 16 + c];
        dv[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, st[s], dv[t], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next query tile overwrites Q / dO
  }

  // Sum the KS partial dV^T tiles ([d][key], rows d = 16 t + 4 g + i) in wave
  // order; thread (d, key) then updates V[key][d].
  float* mine = &qo[wave][0];
#pragma unroll
  for (int t = 0; t < DQ; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mine[(t * 16 + 4 * g + i) * 16 + c] = dv[t][i];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 16 * DP; idx += 64 * KS) {
    const int d = idx >> 4;
    const int kc = idx & 15;
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < KS; ++w) {
      acc += qo[w][idx];
    }
    if (d < D && j0 + kc < S) {
      float* vp = v + static_cast<size_t>(j0 + kc) * D + d;
      *vp = *vp - lr * acc;
    }
  }
}

// loss = sum over n elements of (out - target)^2 * norm, one workgroup,
// fixed reduction order (deterministic).
// Workgroup b sums the squared differences of its contiguous chunk
// [b, b + 1) * chunk (each thread strided through it, eight loads in flight,
// then a tree over the threads) and stores the partial; the last workgroup to
// finish (device-scope counter, reset by it) adds the partials in workgroup
// order.  The same n and grid always give the same bits.
__global__ __launch_bounds__(1024) void mse_loss_kernel(const float* __restrict__ out,
                                                        const float* __restrict__ target, size_t n, size_t chunk,
                                                        float norm, float* __restrict__ loss,
                                                        float* __restrict__ partials, unsigned* __restrict__ counter) {
  __shared__ float part[1024];
  const size_t lo = static_cast<size_t>(blockIdx.x) * chunk;
  const size_t hi = lo + chunk < n ? lo + chunk : n;
  float acc = 0.0f;
#pragma unroll 8
  for (size_t i = lo + threadIdx.x; i < hi; i += 1024) {
    const float d = out[i] - target[i];
    acc += d * d;
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) {
      part[threadIdx.x] += part[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (gridDim.x == 1) {
    if (threadIdx.x == 0) {
      *loss = part[0] * norm;
    }
    return;
  }
  if (threadIdx.x == 0) {
    __hip_atomic_store(&partials[blockIdx.x], part[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1) {
      float total = 0.0f;
      for (unsigned b = 0; b < gridDim.x; ++b) {
        total += __hip_atomic_load(&partials[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      *loss = total * norm;
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------
// 16-bit: 4 waves x 32 queries per workgroup, 64-key tiles, software
// pipelined.  While a wave turns tile j's scores into probabilities (VALU),
// the MFMAs of tile j+1's scores are already in flight; then tile j's P.V
// MFMAs.  K and V^T tiles reach LDS by direct global -> LDS loads (no staging
// registers, no LDS store instructions), two buffers each: K of tile j+2 and
// V^T of tile j+1 load while tile j is processed; one wait + barrier per tile.
// Q fragments live in registers; v_mfma_f32_32x32x16_{bf16,f16}.
//
// LDS layouts, 16-byte chunks XOR-swizzled so that every fragment read is
// conflict-free (a 16-byte read serves 16 lanes per clock over 64 banks):
//   K tile   [64 keys][D]  rows of 2D bytes: chunk ^ (row & 15) for 256-byte
//                          rows, chunk ^ ((row >> 1) & 7) for 128-byte rows
//   V^T tile [D][64 keys]  128-byte rows: chunk ^ ((row >> 1) & 7)
// Key order: MFMA row m of a 32-key block reads key pi(m), pi swapping bits 2
// and 3 of m.  Accumulator register i of lane l then holds key
// 16*(i/8) + 8*(l/32) + i%8, so the 8 probabilities a lane feeds to one P.V
// MFMA are 8 consecutive keys and its V^T operand is one 16-byte read.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// A 16-bit value as fp32.
template <typename T>
__device__ __forceinline__ float half_bits_to_f32(uint32_t h);
template <>
__device__ __forceinline__ float half_bits_to_f32<BF16>(uint32_t h) {
  return __builtin_bit_cast(float, (h & 0xffffu) << 16);
}
template <>
__device__ __forceinline__ float half_bits_to_f32<F16>(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xffffu)));
}

// Eight packed 16-bit values times c, rounded back (RNE).
template <typename T>
__device__ __forceinline__ u32x4 scale_halves(u32x4 v, float c) {
  u32x4 r;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    r[w] = pack2<T>(half_bits_to_f32<T>(v[w]) * c, half_bits_to_f32<T>(v[w] >> 16) * c);
  }
  return r;
}

// Per-wave state and steps of the 16-bit attention: queries q0 .. q0 + 31
// against 64-key K / V^T tiles in LDS, in the layouts above.  Shared by
// attn_fwd_half_kernel (tiles streamed through two LDS buffers) and
// vit_qkv_attn_kernel (every tile resident), so both compute the same values.
template <typename T, int D>
struct HalfAttnWave {
  static constexpr int KT = 64;
  static constexpr int KCH = D / 8;  // 16-byte chunks per K row
  static constexpr int DT = D / 32;
  static constexpr int QS = D / 16;
  static_assert(D == 64 || D == 128, "head dim");
  u32x4 qf[QS];
  floatx16 o[DT];
  // Scores are kept relative to a per-query reference m_run (exp2 units): the
  // QK^T MFMAs start from -m_run instead of zero, so x = s*c - m_run comes
  // out of the accumulator and p = exp2(x) needs no extra arithmetic.  The
  // reference moves to the tile max on a query's first tile with a valid key,
  // and later only when the max exceeds it by more than 8 (then O, l and the
  // tile's scores are shifted); exponents stay <= 8.
  float m_run;
  float l_run;
  bool started;
  int lrow;
  int half;
  int prow;
  int kswz;
  int vswz;
  int q0;
  int qi;
  int S;
  int causal;

  // qrow: this lane's Q row (query q0 + lane % 32), D contiguous values.  Q
  // fragments are pre-multiplied by c = scale * log2(e) (rounded back to the
  // 16-bit type once per wave), so the QK^T MFMAs produce scores in exp2 units.
  __device__ __forceinline__ void init(const uint16_t* qrow, int q0_, int S_, int causal_, float scale, int lane) {
    lrow = lane & 31;
    half = lane >> 5;
    q0 = q0_;
    qi = q0 + lrow;
    S = S_;
    causal = causal_;
    const float c = scale * kLog2e;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      qf[s] = scale_halves<T>(*reinterpret_cast<const u32x4*>(qrow + s * 16 + 8 * half), c);
    }
    // Fragment addresses (elements).  K: MFMA row lrow of 32-key block kt
    // reads key kt*32 + pi(lrow); its swizzle does not depend on kt.
    prow = (lrow & ~12) | ((lrow & 4) << 1) | ((lrow & 8) >> 1);
    kswz = KCH == 16 ? (prow & 15) : ((prow >> 1) & 7);
    vswz = (lrow >> 1) & 7;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      o[t] = zero16();
    }
    m_run = 0.0f;
    l_run = 0.0f;
    started = false;
  }

  // Raw scores of the K tile at ks (two 32-key blocks).
  __device__ __forceinline__ void qk(const uint16_t* ks, floatx16 (&sc)[2]) const {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      sc[kt] = zero16();
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        const u32x4 a =
            *reinterpret_cast<const u32x4*>(ks + (kt * 32 + prow) * D + (((2 * s + half) ^ kswz) << 3));
        sc[kt] = mfma32x32x16<T>(a, qf[s], sc[kt]);
      }
    }
  }

  // Tile j's probabilities from its raw scores s_cur (p = exp2(s*c - m*c), m
  // the running max of raw scores), with the next tile's QK^T MFMAs (K tile
  // at ksn) in the same basic block so the scheduler interleaves them with the
  // VALU work, then tile j's O^T += V^T . P^T (V^T tile at vs).
  __device__ __forceinline__ void step(int j, const uint16_t* ksn, const uint16_t* vs, floatx16 (&s_cur)[2],
                                       floatx16 (&s_nxt)[2]) {
      const int j0 = j * KT;
      if ((j0 + KT > S) || (causal && j0 + KT - 1 > q0)) {
        // key = j0 + 8*half + off with off a compile-time constant per register;
        // masked when key >= S or (causal) key > qi, i.e. off > lim.
        const int lim = (causal ? min(qi, S - 1) : S - 1) - j0 - 8 * half;
  #pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
  #pragma unroll
          for (int i = 0; i < 16; ++i) {
            if (kt * 32 + 16 * (i >> 3) + (i & 7) > lim) {
              s_cur[kt][i] = kMaskValue;
            }
          }
        }
      }
      float mt = kMaskValue;
  #pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
  #pragma unroll
        for (int i = 0; i < 16; ++i) {
          mt = fmaxf(mt, s_cur[kt][i]);
        }
      }
      mt = max_xor32(mt);
      // Lanes l and l ^ 32 hold the same query and see the same mt, so their
      // references stay equal.  O and l always share the reference, so O/l is
      // unchanged by a shift.
      const bool valid = mt > 0.5f * kMaskValue;
      const bool shift = valid && (!started || mt > 8.0f);
      started = started || valid;
      if (__any(shift)) {
        const float sh = shift ? mt : 0.0f;
        const float alpha = fast_exp2(-sh);
        m_run += sh;
        l_run *= alpha;
  #pragma unroll
        for (int t = 0; t < DT; ++t) {
  #pragma unroll
          for (int i = 0; i < 16; ++i) {
            o[t][i] *= alpha;
          }
        }
  #pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
  #pragma unroll
          for (int i = 0; i < 16; ++i) {
            s_cur[kt][i] -= sh;
          }
        }
      }
      // Phase 1: the 32 exponentials of this lane, packed to 16-bit pairs as
      // they come, with the next tile's 2*QS QK^T MFMAs issued between them
      // (EPM exponentials per MFMA, K fragments read two MFMAs ahead).  The
      // sched_barrier after each group keeps this order: an MFMA runs for 32
      // clocks while the wave issues the group's VALU work behind it.
      constexpr int NQK = 2 * QS;
      constexpr int EPM = 32 / NQK;
      floatx16 negm;
  #pragma unroll
      for (int i = 0; i < 16; ++i) {
        negm[i] = -m_run;
      }
      float ls = 0.0f;
      u32x4 pb[4];
      auto kfrag = [&](int g) {
        const int kt = g / QS;
        const int s = g - kt * QS;
        return *reinterpret_cast<const u32x4*>(ksn + (kt * 32 + prow) * D + (((2 * s + half) ^ kswz) << 3));
      };
      // Fragments rotate through a 3-entry ring indexed by the unrolled g
      // (no register copies).
      u32x4 kf[3];
      kf[0] = kfrag(0);
      kf[1] = kfrag(1);
  #pragma unroll
      for (int g = 0; g < NQK; ++g) {
        if (g + 2 < NQK) {
          kf[(g + 2) % 3] = kfrag(g + 2);
        }
        {
          const int kt = g / QS;
          const int s = g - kt * QS;
          s_nxt[kt] = mfma32x32x16<T>(kf[g % 3], qf[s], s == 0 ? negm : s_nxt[kt]);
        }
  #pragma unroll
        for (int e = 0; e < EPM; e += 2) {
          const int idx = g * EPM + e;  // score element idx and idx + 1
          const float p0 = fast_exp2(s_cur[idx >> 4][idx & 15]);
          const float p1 = fast_exp2(s_cur[idx >> 4][(idx & 15) + 1]);
          const uint32_t pair = pack2<T>(p0, p1);
          // l sums the rounded probabilities the P.V MFMAs consume.
          ls = add_pair<T>(pair, ls);
          pb[idx >> 3][(idx & 7) >> 1] = pair;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      l_run += ls;
      // Phase 2: O^T += V^T . P^T, V^T fragments read two MFMAs ahead.
      auto vfrag = [&](int g) {
        const int ks2 = g / DT;
        const int t = g - ks2 * DT;
        return *reinterpret_cast<const u32x4*>(vs + (t * 32 + lrow) * KT + (((2 * ks2 + half) ^ vswz) << 3));
      };
      constexpr int NPV = 4 * DT;
      u32x4 vf[3];
      vf[0] = vfrag(0);
      vf[1] = vfrag(1);
  #pragma unroll
      for (int g = 0; g < NPV; ++g) {
        if (g + 2 < NPV) {
          vf[(g + 2) % 3] = vfrag(g + 2);
        }
        const int ks2 = g / DT;
        const int t = g - ks2 * DT;
        o[t] = mfma32x32x16<T>(vf[g % 3], pb[ks2], o[t]);
        __builtin_amdgcn_sched_barrier(0);
      }
  }

  // Normalises and stores this wave's rows: fp32 [bh][S][D] to O, or (O null)
  // 16-bit heads-concatenated [b][S][heads * D] to Ocat.
  __device__ __forceinline__ void store(float* __restrict__ O, uint16_t* __restrict__ Ocat, int bh, int heads) const {
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = 1.0f / l_tot;
    if (qi >= S) {
      return;
    }
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
};

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void attn_fwd_half_kernel(const uint16_t* __restrict__ Q,
                                                               const uint16_t* __restrict__ K,
                                                               const uint16_t* __restrict__ Vt, float* __restrict__ O,
                                                               uint16_t* __restrict__ Ocat, int heads, int S,
                                                               int S_pad, int causal, float scale) {
  constexpr int KT = 64;
  constexpr int KCH = D / 8;               // 16-byte chunks per K row
  constexpr int K_RPI = 64 / KCH;          // K rows per 1 KB load instruction
  constexpr int TILE = KT * D;             // elements of a K (or V^T) tile
  constexpr int LPW = TILE * 2 / 1024 / 4; // load instructions per wave per operand
  // One LDS array: K buffers at 0 and TILE, V^T buffers at 2*TILE and
  // 3*TILE (copies address it by byte offset from its base).
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nqb = S_pad / 128;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.y);  // heaviest (causal) blocks first
  const int bh = blockIdx.x;
  const int q0 = qb * 128 + wave * 32;
  const size_t hoff = static_cast<size_t>(bh) * S_pad * D;
  const uint16_t* Qh = Q + hoff;

  // Load mapping: wave w issues instructions w + 4j (j < LPW) of each operand.
  // K instruction i fills rows K_RPI*i + lane / KCH, physical chunk lane % KCH;
  // V^T instruction i fills rows 8i + lane / 8, physical chunk lane % 8.
  // Per-lane byte offsets are 32-bit (the host keeps a head below 2^30
  // elements) and fixed; the tile base is uniform, so every copy takes the
  // scalar-base form (load_lds16_sbase) with one M0 move of setup.
  const uint16_t* Kh = K + hoff;
  const uint16_t* Vh = Vt + hoff;
  uint32_t k_off[LPW];
  uint32_t v_off[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int ins = wave + 4 * j;
    const int kr = K_RPI * ins + lane / KCH;
    const int kswz = KCH == 16 ? (kr & 15) : ((kr >> 1) & 7);
    k_off[j] = static_cast<uint32_t>(kr * D + ((lane % KCH) ^ kswz) * 8) * 2u;
    const int vr = 8 * ins + (lane >> 3);
    v_off[j] = static_cast<uint32_t>(vr * S_pad + ((lane & 7) ^ ((vr >> 1) & 7)) * 8) * 2u;
  }
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = lds_addr(smem);
  auto issue_k = [&](int buf, int tile) {
    const uint16_t* base = Kh + static_cast<size_t>(tile) * KT * D;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      load_lds16_sbase(k_off[j], base, lds0 + 2u * static_cast<uint32_t>(buf * TILE + (wave_s + 4 * j) * 512));
    }
  };
  auto issue_v = [&](int buf, int tile) {
    const uint16_t* base = Vh + tile * KT;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      load_lds16_sbase(v_off[j], base, lds0 + 2u * static_cast<uint32_t>((2 + buf) * TILE + (wave_s + 4 * j) * 512));
    }
  };

  HalfAttnWave<T, D> w;
  w.init(Qh + static_cast<size_t>(q0 + (lane & 31)) * D, q0, S, causal, scale, lane);
  const int kend = causal ? min(S, qb * 128 + 128) : S;
  const int nt = (kend + KT - 1) / KT;
  // Causal: tile j is skipped by a wave whose queries all precede its keys
  // (monotone in j: a skipped tile is followed only by skipped tiles).
  auto active = [&](int j) { return !(causal && j * KT > q0 + 31); };

  floatx16 s_a[2];
  floatx16 s_b[2];
  issue_k(0, 0);
  issue_v(0, 0);
  if (nt > 1) {
    issue_k(1, 1);
  }
  wait_vmcnt<0>();
  stage_barrier();
  w.qk(smem, s_a);   // tile 0 is active for every wave
  stage_barrier();   // K buffer 0 is refilled next
  // One tile: its loads of K(j+2) and V^T(j+1) go out first, then the
  // pipelined step (the next tile's scores are computed unconditionally, one
  // code path; past the last tile, or when the next tile is skipped, they
  // come from a stale but stable K buffer and go unused), then the wait and
  // barrier.  Unrolled by two so the score registers swap roles instead of
  // being copied.
  auto tile = [&](int j, floatx16 (&s_cur)[2], floatx16 (&s_nxt)[2]) {
    if (j + 2 < nt) {
      issue_k(j & 1, j + 2);
    }
    if (j + 1 < nt) {
      issue_v((j + 1) & 1, j + 1);
    }
    if (active(j)) {
      w.step(j, smem + ((j + 1) & 1) * TILE, smem + (2 + (j & 1)) * TILE, s_cur, s_nxt);
    }
    wait_vmcnt<0>();  // this wave's loads of K(j+2) and V^T(j+1) have landed
    stage_barrier();  // everyone's have; everyone is done with K(j+1) and V^T(j)
  };
  for (int j = 0; j < nt; j += 2) {
    tile(j, s_a, s_b);
    if (j + 1 < nt) {
      tile(j + 1, s_b, s_a);
    }
  }
  w.store(O, Ocat, bh, heads);
}

// ---------------------------------------------------------------------------
// ViT block: the QKV projection of one (image, head) fused with its
// attention, so Q, K and V^T never leave LDS.  T <= 224 tokens (nrb =
// ceil(T/32) <= 7 blocks of 32), head dim 64.  Each (image b, head h) takes
// nparts = min(2, nrb) workgroups of 8 waves; part p owns a contiguous range
// of query blocks [qlo, qhi) (at most 4), and every part projects K and V for
// all tokens (the attention of its queries needs every key), Q only for its
// own queries.
//  1. Projection: token rows of image b times the head's 192 rows of W_qkv^T
//     (Q rows h*64.., K rows E + h*64.., V rows 2E + h*64..), in 64-deep
//     stages through a ring of three LDS buffers: 224 token rows (rows past T
//     re-read token T-1, so every value stays finite) and the 192 weight
//     rows, 128-byte rows with chunk ^ ((row >> 1) & 7), one direct
//     global -> LDS copy per 8 rows (52 per stage, 6 or 7 per wave).  The
//     copies of stage s+2 go out during stage s, two after each k-step.
//     32x32 output blocks ("units") per wave: wave w < nrb takes K and V of
//     token block w (four units) and, when w is one of this part's query
//     blocks, Q's first 32 columns; Q's other 32 columns of this part's first
//     min(3, #query blocks) blocks go to wave 7 and those of the rest stay
//     with their wave (at T = 196 that is 9 units on every SIMD).  Q and K
//     units compute W . tokens^T (rows d, columns tokens) and V units
//     tokens . W^T, so every lane ends up with 4 consecutive elements of one
//     LDS row below.  v_mfma_f32_32x32x16 in the k order of the QKV GEMM, the
//     fragments of k-step kk+1 read while kk's MFMAs run.
//  2. The accumulators go to LDS as 16-bit Q [128][64] (this part's queries),
//     K tiles [64][64] and V^T tiles [64][64] (keys past the last token block
//     zero) in attn_fwd_half_kernel's layouts, 8-byte stores.
//  3. Wave a < #query blocks runs attention for query block qlo + a over
//     every key tile (HalfAttnWave: attn_fwd_half_kernel's arithmetic) and
//     stores its rows of the heads-concatenated output.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(512) void vit_qkv_attn_kernel(const uint16_t* __restrict__ tokens,
                                                          const uint16_t* __restrict__ Wqkv_t,
                                                          uint16_t* __restrict__ Ocat, int T_, int E, int H,
                                                          int nparts, int tb, int th, float scale) {
  constexpr int D = 64;
  constexpr int KT = 64;
  constexpr int TILE = KT * D;            // elements of a K (or V^T) tile
  constexpr int AR = 224;                 // token rows per stage (padded)
  constexpr int WR = 3 * D;               // weight rows: Q, K, V of one head
  constexpr int NB = 3;                   // ring buffers
  constexpr int STAGE = (AR + WR) * 64;   // elements per projection stage
  constexpr int NCP = (AR + WR) / 8;      // 1 KB copies per stage (52)
  constexpr int CPW = (NCP + 7) / 8;      // per wave, at most (7)
  constexpr int ACP = AR / 8;             // ... of token rows (28)
  constexpr int QR = 128;                 // Q rows held (4 query blocks)
  constexpr int SP = 256;                 // keys held by the K / V^T tiles
  // Phase 2 layout (elements): Q [QR][D] at 0, then the K tiles, then the
  // V^T tiles.
  constexpr int KOFF = QR * D;
  constexpr int VOFF = KOFF + (SP / KT) * TILE;
  static_assert(VOFF + (SP / KT) * TILE <= NB * STAGE, "phase 2 fits in the projection ring");
  static_assert(NB * STAGE * 2 <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) uint16_t smem[NB * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  // Workgroup -> (image, head, part).  With tb > 0 the 8 XCDs (workgroup w
  // runs on XCD w % 8) each take a tb x th block of (image, head) pairs, so
  // an XCD's L2 fetches the tokens of tb images and the weights of th heads
  // (the host picks the block that minimises those bytes); else in order.
  int b;
  int h;
  int part;
  if (tb > 0) {
    const int x = blockIdx.x & 7;
    const int l = blockIdx.x >> 3;
    const int tiles_b = static_cast<int>(gridDim.x) / (H * nparts) / tb;
    part = l % nparts;
    const int r = l / nparts;
    b = (x % tiles_b) * tb + r % tb;
    h = (x / tiles_b) * th + r / tb;
  } else {
    const int q = blockIdx.x / nparts;
    part = blockIdx.x - q * nparts;
    b = q / H;
    h = q - b * H;
  }
  const int bh = b * H + h;
  const uint16_t* tok = tokens + static_cast<size_t>(b) * T_ * E;
  const int nrb = (T_ + 31) >> 5;
  const int per = (nrb + nparts - 1) / nparts;
  const int qlo = part * per;
  const int nq = min(nrb, qlo + per) - qlo;  // 1..4
  const int nmove = min(3, nq);              // Q column-block-1 units done by wave 7

  // Copy j of this wave is instruction i = wave + 8j of the stage (i < NCP):
  // stage rows 8i + lane/8 (token rows for i < ACP, weight rows after),
  // physical chunk lane % 8 holding logical chunk (lane % 8) ^ ((row >> 1) & 7).
  // Byte offsets are 32-bit (the host keeps T*E*2 and 3*E*E*2 below 2^31).
  uint32_t off[CPW];
  const uint16_t* cbase[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int i = wave_s + 8 * j;
    const int row = 8 * i + (lane >> 3);
    const int lch = (lane & 7) ^ ((row >> 1) & 7);
    if (i < ACP) {
      const int t = min(row, T_ - 1);
      off[j] = static_cast<uint32_t>(t * E + lch * 8) * 2u;
      cbase[j] = tok;
    } else {
      const int r = min(row - AR, WR - 1);
      const int wrow = (r >> 6) * E + h * D + (r & 63);
      off[j] = static_cast<uint32_t>(wrow * E + lch * 8) * 2u;
      cbase[j] = Wqkv_t;
    }
  }
  const bool full_cpw = wave_s + 8 * (CPW - 1) < NCP;  // CPW copies per stage, else CPW - 1
  const uint32_t lds0 = lds_addr(smem);
  // Copies j0 .. j1-1 of stage st into ring slot buf.
  auto issue = [&](int st, int buf, int j0, int j1) {
    const int k0 = st * 64;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      if (j >= j0 && j < j1 && (j < CPW - 1 || full_cpw)) {
        load_lds16_sbase(off[j], cbase[j] + k0,
                         lds0 + 2u * static_cast<uint32_t>(buf * STAGE + (wave_s + 8 * j) * 512));
      }
    }
  };

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  // Token rows 32w + lrow and weight rows AR + 32cb + lrow share the swizzle
  // (lrow >> 1) & 7.
  const int swz = (lrow >> 1) & 7;
  floatx16 acc[6];
#pragma unroll
  for (int u = 0; u < 6; ++u) {
    acc[u] = zero16();
  }
  // Wave roles (uniform): main waves w < nrb hold K0 K1 V0 V1 in acc[0..3],
  // Q0 in acc[4] when w is a query block of this part, and Q1 in acc[5] when
  // it is one past the first nmove; wave 7 holds Q1 of query blocks
  // qlo .. qlo + nmove - 1 in acc[0..nmove-1].
  const bool main_w = wave_s < nrb;
  const bool has_q = main_w && wave_s >= qlo && wave_s < qlo + nq;
  const bool own_q1 = has_q && wave_s - qlo >= nmove;
  const bool helper = wave_s == 7;

  // The stage loop; compute(sb, cp) runs this wave's 4 k-steps on the stage
  // at sb and calls cp(kk) after k-step kk's MFMAs, which issues two of the
  // copies of stage st + 2 (the last k-step the rest): spread over the stage,
  // the copies do not queue up behind each other at the address unit while
  // the MFMAs wait.
  const int nst = E / 64;
  auto run = [&](auto compute) {
    issue(0, 0, 0, CPW);
    if (nst > 1) {
      issue(1, 1, 0, CPW);
    }
    int buf = 0;   // ring slot of stage st
    int buf2 = 2;  // ring slot of stage st + 2
    for (int st = 0; st < nst; ++st) {
      // This wave's copies of stage st have landed (those of st + 1 may still
      // be in flight), then everyone's have, and everyone is done with stage
      // st - 1, whose slot takes stage st + 2.
      if (st + 1 < nst) {
        if (full_cpw) {
          wait_vmcnt<CPW>();
        } else {
          wait_vmcnt<CPW - 1>();
        }
      } else {
        wait_vmcnt<0>();
      }
      stage_barrier();
      const bool more = st + 2 < nst;
      auto cp = [&](int kk) {
        if (more) {
          issue(st + 2, buf2, 2 * kk, kk == 3 ? CPW : 2 * kk + 2);
        }
      };
      compute(smem + buf * STAGE, cp);
      buf = buf == NB - 1 ? 0 : buf + 1;
      buf2 = buf2 == NB - 1 ? 0 : buf2 + 1;
    }
  };
  auto rd_a = [&](const uint16_t* sb, int kk, int rb) {
    return *reinterpret_cast<const u32x4*>(sb + (rb * 32 + lrow) * 64 + (((2 * kk + lhalf) ^ swz) << 3));
  };
  auto rd_w = [&](const uint16_t* sb, int kk, int cb) {
    return *reinterpret_cast<const u32x4*>(sb + (AR + cb * 32 + lrow) * 64 + (((2 * kk + lhalf) ^ swz) << 3));
  };
  // Main waves: NQ = 0, 1 or 2 Q units.  Fragment slots: [0] tokens, [1..4]
  // K0 K1 V0 V1 weights, [5..] Q0 Q1 weights.
  auto main_stage = [&](auto nq_c) {
    constexpr int NQ = decltype(nq_c)::value;
    constexpr int NF = 5 + NQ;
    return [&](const uint16_t* sb, auto cp) {
      u32x4 f[2][NF];
      auto rd = [&](int kk, u32x4 (&g)[NF]) {
        g[0] = rd_a(sb, kk, wave_s);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          g[1 + u] = rd_w(sb, kk, 2 + u);
        }
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
          g[5 + u] = rd_w(sb, kk, u);
        }
      };
      rd(0, f[0]);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk < 3) {
          rd(kk + 1, f[(kk + 1) & 1]);
        }
        const u32x4(&g)[NF] = f[kk & 1];
        acc[0] = mfma32x32x16<T>(g[1], g[0], acc[0]);  // K rows d 0..31
        acc[1] = mfma32x32x16<T>(g[2], g[0], acc[1]);  // K rows d 32..63
        acc[2] = mfma32x32x16<T>(g[0], g[3], acc[2]);  // V columns d 0..31
        acc[3] = mfma32x32x16<T>(g[0], g[4], acc[3]);  // V columns d 32..63
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
          acc[4 + u] = mfma32x32x16<T>(g[5 + u], g[0], acc[4 + u]);  // Q rows d 32u..
        }
        cp(kk);
      }
    };
  };
  // Wave 7: Q1 of NM query blocks.  Fragment slots: [0] Q1 weights, [1..NM]
  // tokens of blocks qlo ...
  auto helper_stage = [&](auto nm_c) {
    constexpr int NM = decltype(nm_c)::value;
    return [&](const uint16_t* sb, auto cp) {
      u32x4 f[2][1 + NM];
      auto rd = [&](int kk, u32x4 (&g)[1 + NM]) {
        g[0] = rd_w(sb, kk, 1);
#pragma unroll
        for (int u = 0; u < NM; ++u) {
          g[1 + u] = rd_a(sb, kk, qlo + u);
        }
      };
      rd(0, f[0]);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk < 3) {
          rd(kk + 1, f[(kk + 1) & 1]);
        }
        const u32x4(&g)[1 + NM] = f[kk & 1];
#pragma unroll
        for (int u = 0; u < NM; ++u) {
          acc[u] = mfma32x32x16<T>(g[0], g[1 + u], acc[u]);
        }
        cp(kk);
      }
    };
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  if (main_w) {
    if (!has_q) {
      run(main_stage(I0{}));
    } else if (!own_q1) {
      run(main_stage(I1{}));
    } else {
      run(main_stage(I2{}));
    }
  } else if (helper) {
    if (nmove == 1) {
      run(helper_stage(I1{}));
    } else if (nmove == 2) {
      run(helper_stage(I2{}));
    } else {
      run(helper_stage(I3{}));
    }
  } else {
    run([](const uint16_t*, auto cp) {
      cp(0);
      cp(1);
      cp(2);
      cp(3);
    });
  }
  __syncthreads();  // every wave is done with the projection buffers

  // Q, K and V^T to LDS.  In a W . tokens^T unit, register 4g + i of lane l
  // holds d = 32cb + 8g + 4(l/32) + i of token 32rb + l%32; in a tokens . W^T
  // unit, token 32rb + 8g + 4(l/32) + i and d = 32cb + l%32.
  uint16_t* Qs = smem;
  uint16_t* Ks = smem + KOFF;
  uint16_t* Vs = smem + VOFF;
  auto store_q = [&](const floatx16& a, int rb, int cb) {
    const int t = rb * 32 + lrow;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = cb * 32 + 8 * g + 4 * lhalf;
      u32x2 v;
      v[0] = pack2<T>(a[4 * g], a[4 * g + 1]);
      v[1] = pack2<T>(a[4 * g + 2], a[4 * g + 3]);
      *reinterpret_cast<u32x2*>(Qs + (t - qlo * 32) * D + d0) = v;
    }
  };
  if (main_w) {
    const int t = wave_s * 32 + lrow;
    const int r = t & (KT - 1);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = cb * 32 + 8 * g + 4 * lhalf;
        u32x2 v;
        v[0] = pack2<T>(acc[cb][4 * g], acc[cb][4 * g + 1]);
        v[1] = pack2<T>(acc[cb][4 * g + 2], acc[cb][4 * g + 3]);
        *reinterpret_cast<u32x2*>(Ks + (t / KT) * TILE + r * D + (((d0 >> 3) ^ ((r >> 1) & 7)) << 3) + (d0 & 7)) = v;
      }
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int d = cb * 32 + lrow;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int t0 = wave_s * 32 + 8 * g + 4 * lhalf;  // keys t0 .. t0 + 3
        const int r0 = t0 & (KT - 1);
        u32x2 v;
        v[0] = pack2<T>(acc[2 + cb][4 * g], acc[2 + cb][4 * g + 1]);
        v[1] = pack2<T>(acc[2 + cb][4 * g + 2], acc[2 + cb][4 * g + 3]);
        uint16_t* vdst = Vs + (t0 / KT) * TILE + d * KT + (((r0 >> 3) ^ ((d >> 1) & 7)) << 3) + (r0 & 7);
        *reinterpret_cast<u32x2*>(vdst) = v;
      }
    }
    if (has_q) {
      store_q(acc[4], wave_s, 0);
      if (own_q1) {
        store_q(acc[5], wave_s, 1);
      }
    }
  } else if (helper) {
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      if (u < nmove) {
        store_q(acc[u], qlo + u, 1);
      }
    }
    if (nrb & 1) {
      // Keys 32 nrb .. 32 nrb + 31 (the second half of the last key tile):
      // zeros (masked keys, whose V rows must stay finite).  K rows 32..63 of
      // that tile are contiguous; V^T rows d hold them in logical chunks 4..7.
      const int tl = nrb >> 1;
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = lane + 64 * q;  // 0..255
        *reinterpret_cast<u32x4*>(Ks + tl * TILE + 32 * D + 8 * c) = z;
        const int d = c >> 2;
        const int lc = 4 + (c & 3);
        *reinterpret_cast<u32x4*>(Vs + tl * TILE + d * KT + ((lc ^ ((d >> 1) & 7)) << 3)) = z;
      }
    }
  }
  __syncthreads();

  if (wave < nq) {
    const int q0 = (qlo + wave) * 32;
    HalfAttnWave<T, D> w;
    w.init(Qs + (wave * 32 + lrow) * D, q0, T_, 0, scale, lane);
    const int nt = (T_ + KT - 1) / KT;
    floatx16 s_a[2];
    floatx16 s_b[2];
    w.qk(Ks, s_a);
    // Every tile is resident: no loads or barriers between tiles.  Past the
    // last tile the next tile's scores come from the last K tile and go
    // unused.
    for (int j = 0; j < nt; j += 2) {
      w.step(j, Ks + min(j + 1, nt - 1) * TILE, Vs + j * TILE, s_a, s_b);
      if (j + 1 < nt) {
        w.step(j + 1, Ks + min(j + 2, nt - 1) * TILE, Vs + (j + 1) * TILE, s_b, s_a);
      }
    }
    w.store(nullptr, Ocat, bh, H);
  }
}

}  // namespace lchip::k

namespace lchip::kern {

using namespace lchip::k;

bool attentionF32Q16Fits(int D, const float* k, const float* v, const float* q) {
  return D <= 64 && D % 4 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(v) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0;
}

int attentionF32DefaultSplits(int bh, int S, int D) {
  if (D <= 64 && D % 4 == 0 && bh * ((S + 15) / 16) <= 256 && S <= 1024) {
    return kAttnF32Q16;
  }
  return attentionF32Splits(bh, S, D, 0);
}

int attentionF32Splits(int bh, int S, int D, int requested) {
  const int nqb = (S + 31) / 32;
  const int dt = (D + 31) / 32;
  if (requested == kAttnF32Q16 && D <= 64 && D % 4 == 0) {
    return kAttnF32Q16;
  }
  // Per-wave K + V tiles must fit the 160 KB of LDS: up to 8 splits at
  // DT <= 2 (140 KB), 2 at DT <= 4, 1 beyond (the launch switches below).
  const int cap = dt <= 2 ? 8 : (dt <= 4 ? 2 : 1);
  if (requested > 0) {
    int ks = 1;
    while (ks * 2 <= requested && ks * 2 <= cap) {
      ks *= 2;
    }
    return ks;
  }
  // Heuristic: enough waves for about two per CU, at most one split per
  // 32-key tile.
  int ks = 1;
  while (ks < cap && static_cast<long long>(nqb) * bh * ks * 2 <= 512 && ks * 2 <= nqb) {
    ks *= 2;
  }
  return ks;
}

namespace {

// 32-key tiles per key split of the 32-query kernel, 0 for none: while its
// grid (query blocks x heads) covers fewer than half the CUs, the key tiles
// of a block are divided among up to 16 workgroups (a power of two, grid at
// most 256 workgroups, every wave still with at least one tile).
int keySplitTiles(int bh, int S, int ks) {
  const int nqb = (S + 31) / 32;
  const long long base = static_cast<long long>(nqb) * bh;
  if (base >= 128) {
    return 0;
  }
  int n = 1;
  while (n < 16 && base * (2 * n) <= 256 && 2LL * n * ks <= nqb) {
    n *= 2;
  }
  return n > 1 ? (nqb + n - 1) / n : 0;
}

// The q16 kernel would serve this call (its pointer-alignment condition aside).
bool q16Serves(int bh, int S, int D, int splits) {
  return (splits == kAttnF32Q16 || (splits == 0 && attentionF32DefaultSplits(bh, S, D) == kAttnF32Q16)) &&
         D <= 64 && D % 4 == 0;
}

}  // namespace

size_t attentionF32WorkspaceFloats(int bh, int S, int D, int splits) {
  if (D <= 0 || D > 256 || S <= 0 || bh <= 0 || q16Serves(bh, S, D, splits)) {
    return 0;
  }
  const int ks = attentionF32Splits(bh, S, D, splits == kAttnF32Q16 ? 0 : splits);
  const int tiles = keySplitTiles(bh, S, ks);
  if (tiles == 0) {
    return 0;
  }
  const int nqb = (S + 31) / 32;
  const size_t nsplit = static_cast<size_t>((nqb + tiles - 1) / tiles);
  return nsplit * static_cast<size_t>(bh) * S * (D + 2);
}

hipError_t attentionF32(const float* q, const float* k, const float* v, float* out, int bh, int S, int D, bool causal,
                        float post_scale, float post_bias, int post_relu, float* stats, hipStream_t stream,
                        int splits, unsigned* done_count, unsigned* done_flag, unsigned done_seq, float* split_ws,
                        size_t split_ws_floats) {
  const DoneFlag done{done_count, done_flag, done_seq};
  if (D <= 0 || D > 256 || S <= 0 || bh <= 0 || (done_flag != nullptr && stats != nullptr)) {
    return hipErrorInvalidValue;
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(D));
  const int cz = causal ? 1 : 0;
  // The 16-query kernel when asked for, and by default while its grid is at
  // most one workgroup per CU (bh * S/16 <= 256, S <= 1024): measured at one
  // head, S = 128 ... 1024, D = 32 / 64, 17-38% faster than the best split of
  // the 32-query kernel.
  const bool dflt = splits == 0 && attentionF32DefaultSplits(bh, S, D) == kAttnF32Q16;
  if ((splits == kAttnF32Q16 || dflt) && attentionF32Q16Fits(D, k, v, q)) {
    const dim3 grid16((S + 15) / 16, bh);
    const AttnSrcGlobal gsrc{q, k, v, done};
    // 8 waves up to S = 256 (each walks at most two 16-key tiles, and the
    // cross-wave merge halves), 16 beyond.  Measured at one head and at 4-16
    // heads, D = 32 / 64: S = 64 5.4 -> 4.7 us, 128 6.0 -> 5.5, 256 7.8 ->
    // 7.2; at S = 512 equal, at 1024 16 waves are 7% faster.
#define LC_ATTN_Q16(DQ_, KS_)                                                                                       \
  hipLaunchKernelGGL((attn_fwd_f32_q16_kernel<DQ_, KS_, AttnSrcGlobal>), grid16, dim3(64 * (KS_)), 0, stream, gsrc, \
                     out, stats, S, D, cz, scale, post_scale, post_bias, post_relu)
    const bool ks8 = S <= 256;
    switch ((D + 15) / 16) {
      case 1: if (ks8) { LC_ATTN_Q16(1, 8); } else { LC_ATTN_Q16(1, 16); } break;
      case 2: if (ks8) { LC_ATTN_Q16(2, 8); } else { LC_ATTN_Q16(2, 16); } break;
      case 3: if (ks8) { LC_ATTN_Q16(3, 8); } else { LC_ATTN_Q16(3, 16); } break;
      default: if (ks8) { LC_ATTN_Q16(4, 8); } else { LC_ATTN_Q16(4, 16); } break;
    }
#undef LC_ATTN_Q16
    return hipGetLastError();
  }
  const int nqb = (S + 31) / 32;
  const int dt = (D + 31) / 32;
  const int ks = attentionF32Splits(bh, S, D, splits == kAttnF32Q16 ? 0 : splits);
  // Key split when the caller's workspace holds the partials; the combine
  // kernel then writes out / stats and raises the completion flag.
  int split_tiles = keySplitTiles(bh, S, ks);
  const int nsplit = split_tiles > 0 ? (nqb + split_tiles - 1) / split_tiles : 1;
  const size_t need = static_cast<size_t>(nsplit) * bh * S * (D + 2);
  if (split_tiles > 0 && (split_ws == nullptr || split_ws_floats < need)) {
    split_tiles = 0;
  }
  const bool split = split_tiles > 0;
  const dim3 grid(nqb, bh, split ? nsplit : 1);
  const bool vec = D % 4 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0;
  const AttnSrcGlobal src{q, k, v, split ? DoneFlag{} : done};
  float* const stats_main = split ? nullptr : stats;
#define LC_ATTN_F32(DT_, KS_)                                                                                       \
  if (vec) {                                                                                                        \
    hipLaunchKernelGGL((attn_fwd_f32_kernel<DT_, KS_, true, AttnSrcGlobal>), grid, dim3(64 * (KS_)), 0,            \
                       stream, src, out, stats_main, S, D, cz, scale, post_scale, post_bias, post_relu,           \
                       split_tiles, split_ws);                                                                      \
  } else {                                                                                                          \
    hipLaunchKernelGGL((attn_fwd_f32_kernel<DT_, KS_, false, AttnSrcGlobal>), grid, dim3(64 * (KS_)), 0, stream,   \
                       src, out, stats_main, S, D, cz, scale, post_scale, post_bias, post_relu, split_tiles,      \
                       split_ws);                                                                                   \
  }
#define LC_ATTN_F32_KS(DT_)                                                                                         \
  switch (ks) {                                                                                                     \
    case 8: LC_ATTN_F32(DT_, (DT_ <= 2 ? 8 : 1)); break;                                                            \
    case 4: LC_ATTN_F32(DT_, (DT_ <= 2 ? 4 : 1)); break;                                                            \
    case 2: LC_ATTN_F32(DT_, (DT_ <= 4 ? 2 : 1)); break;                                                            \
    default: LC_ATTN_F32(DT_, 1); break;                                                                            \
  }
  switch (dt) {
    case 1: LC_ATTN_F32_KS(1); break;
    case 2: LC_ATTN_F32_KS(2); break;
    case 3: LC_ATTN_F32_KS(3); break;
    case 4: LC_ATTN_F32_KS(4); break;
    case 5: LC_ATTN_F32(5, 1); break;
    case 6: LC_ATTN_F32(6, 1); break;
    case 7: LC_ATTN_F32(7, 1); break;
    default: LC_ATTN_F32(8, 1); break;
  }
#undef LC_ATTN_F32_KS
#undef LC_ATTN_F32
  if (split) {
    const int rows = bh * S;
    hipLaunchKernelGGL(attn_split_combine_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, split_ws, out, stats,
                       rows, D, nsplit, post_scale, post_bias, post_relu, done);
  }
  return hipGetLastError();
}

bool convAttentionStagesInputs(int batch, int cin, int h, int wd, int cout, int kh, int kw, int sh, int sw, int ph,
                               int pw) {
  const int oh = (h + 2 * ph - kh) / sh + 1;
  const int ow = (wd + 2 * pw - kw) / sw + 1;
  const long long n = static_cast<long long>(batch) * cout * oh * ow;
  const long long xs = static_cast<long long>(batch) * cin * h * wd;
  const long long ws = static_cast<long long>(cout) * cin * kh * kw;
  return n + xs + ws + cout <= AttnSrcConvRepeat::kLds;
}

hipError_t convAttentionF32(const float* x, const float* w, const float* bias, int batch, int cin, int h, int wd,
                            int cout, int kh, int kw, int sh, int sw, int ph, int pw, int S, int D, float* out,
                            hipStream_t stream, unsigned* done_count, unsigned* done_flag, unsigned done_seq) {
  const int oh = (h + 2 * ph - kh) / sh + 1;
  const int ow = (wd + 2 * pw - kw) / sw + 1;
  const long long n = static_cast<long long>(batch) * cout * oh * ow;
  if (D <= 0 || D > 256 || S <= 0 || n <= 0 || n > AttnSrcConvRepeat::kOut ||
      3LL * S * D >= (1LL << 31)) {
    return hipErrorInvalidValue;
  }
  const long long xs = static_cast<long long>(batch) * cin * h * wd;
  const long long ws = static_cast<long long>(cout) * cin * kh * kw;
  const int big = 1 << 30;  // sizes beyond LDS staging just disable it
  AttnSrcConvRepeat src{x, w, bias, cin, h, wd, cout, kh, kw, sh, sw, ph, pw, oh, ow, static_cast<int>(n),
                        static_cast<int>(xs < big ? xs : big), static_cast<int>(ws < big ? ws : big),
                        static_cast<size_t>(S) * D};
  src.done = DoneFlag{done_count, done_flag, done_seq};
  const float scale = 1.0f / sqrtf(static_cast<float>(D));
  // D <= 64: the 16-query kernel (16 waves of 16-key tiles, 8 at D > 48 so
  // that the per-wave tiles fit next to the conv buffer).
  if (D <= 64) {
    const dim3 grid16((S + 15) / 16, 1);
#define LC_CA_Q16(DQ_, KS_)                                                                                         \
  hipLaunchKernelGGL((attn_fwd_f32_q16_kernel<DQ_, KS_, AttnSrcConvRepeat>), grid16, dim3(64 * (KS_)), 0, stream,   \
                     src, out, nullptr, S, D, 0, scale, 1.0f, 0.0f, 0)
    switch ((D + 15) / 16) {
      case 1: LC_CA_Q16(1, 16); break;
      case 2: LC_CA_Q16(2, 16); break;
      case 3: LC_CA_Q16(3, 16); break;
      default: LC_CA_Q16(4, 8); break;
    }
#undef LC_CA_Q16
    return hipGetLastError();
  }
  const int nqb = (S + 31) / 32;
  const dim3 grid(nqb, 1);
  const int dt = (D + 31) / 32;
  // Key splits as for attentionF32, within LDS next to the 48 KB conv buffer.
  int ks = 1;
  while (ks < 4 && nqb * ks * 2 <= 512 && ks * 2 <= nqb && (ks * 2) * dt <= 8) {
    ks *= 2;
  }
#define LC_CA_F32(DT_, KS_)                                                                                         \
  hipLaunchKernelGGL((attn_fwd_f32_kernel<DT_, KS_, false, AttnSrcConvRepeat>), grid, dim3(64 * (KS_)), 0, stream, \
                     src, out, nullptr, S, D, 0, scale, 1.0f, 0.0f, 0, 0, nullptr)
#define LC_CA_F32_KS(DT_)                                                                                           \
  switch (ks) {                                                                                                     \
    case 4: LC_CA_F32(DT_, (DT_ <= 2 ? 4 : 1)); break;                                                              \
    case 2: LC_CA_F32(DT_, (DT_ <= 4 ? 2 : 1)); break;                                                              \
    default: LC_CA_F32(DT_, 1); break;                                                                              \
  }
  switch (dt) {
    case 1: LC_CA_F32_KS(1); break;
    case 2: LC_CA_F32_KS(2); break;
    case 3: LC_CA_F32_KS(3); break;
    case 4: LC_CA_F32_KS(4); break;
    case 5: LC_CA_F32(5, 1); break;
    case 6: LC_CA_F32(6, 1); break;
    case 7: LC_CA_F32(7, 1); break;
    default: LC_CA_F32(8, 1); break;
  }
#undef LC_CA_F32_KS
#undef LC_CA_F32
  return hipGetLastError();
}

size_t attentionDvWorkspaceFloats(int bh, int S, int D, int splits) {
  if (D <= 0 || D > 256 || S <= 0 || bh <= 0 || q16Serves(bh, S, D, splits)) {
    return 0;
  }
  const int ks = attentionF32Splits(bh, S, D, splits == kAttnF32Q16 ? 0 : splits);
  const int tiles = keySplitTiles(bh, S, ks);
  if (tiles == 0) {
    return 0;
  }
  const int nqt = (S + 31) / 32;
  return static_cast<size_t>((nqt + tiles - 1) / tiles) * bh * S * D;
}

hipError_t attentionDvUpdateF32(const float* q, const float* k, float* v, const float* out, const float* target,
                                const float* stats, int bh, int S, int D, bool causal, float lr,
                                hipStream_t stream, int splits, float* split_ws, size_t split_ws_floats) {
  if (D <= 0 || D > 256 || S <= 0 || bh <= 0) {
    return hipErrorInvalidValue;
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(D));
  const int cz = causal ? 1 : 0;
  // The 16-key-block kernel under the forward's rule (asked for, or by
  // default while its grid is at most one workgroup per CU).
  const bool dflt = splits == 0 && attentionF32DefaultSplits(bh, S, D) == kAttnF32Q16;
  const bool aligned = reinterpret_cast<uintptr_t>(out) % 16 == 0 && reinterpret_cast<uintptr_t>(target) % 16 == 0;
  if ((splits == kAttnF32Q16 || dflt) && aligned && attentionF32Q16Fits(D, k, v, q)) {
    const dim3 grid16((S + 15) / 16, bh);
#define LC_DV_Q16(DQ_)                                                                                              \
  hipLaunchKernelGGL((attn_dv_f32_q16_kernel<DQ_, 16>), grid16, dim3(1024), 0, stream, q, k, v, out, target, stats, \
                     S, D, cz, scale, lr)
    switch ((D + 15) / 16) {
      case 1: LC_DV_Q16(1); break;
      case 2: LC_DV_Q16(2); break;
      case 3: LC_DV_Q16(3); break;
      default: LC_DV_Q16(4); break;
    }
#undef LC_DV_Q16
    return hipGetLastError();
  }
  const int nkb = (S + 31) / 32;
  const int dt = (D + 31) / 32;
  // Query-tile splits: the same rule and LDS limits as the forward's key
  // splits (K tile + per-wave Q / dO tiles).
  const int ks = attentionF32Splits(bh, S, D, splits == kAttnF32Q16 ? 0 : splits);
  // Small grids also divide each key block's query tiles among workgroups
  // (the forward's rule), when the caller's workspace holds the partials.
  int split_qt = keySplitTiles(bh, S, ks);
  const int nsplit = split_qt > 0 ? (nkb + split_qt - 1) / split_qt : 1;
  if (split_qt > 0 && (split_ws == nullptr || split_ws_floats < static_cast<size_t>(nsplit) * bh * S * D)) {
    split_qt = 0;
  }
  const dim3 grid(nkb, bh, split_qt > 0 ? nsplit : 1);
#define LC_DV_F32(DT_, KS_)                                                                                         \
  hipLaunchKernelGGL((attn_dv_f32_kernel<DT_, KS_>), grid, dim3(64 * (KS_)), 0, stream, q, k, v, out, target, stats, \
                     S, D, cz, scale, lr, split_qt, split_ws)
#define LC_DV_F32_KS(DT_)                                                                                           \
  switch (ks) {                                                                                                     \
    case 8: LC_DV_F32(DT_, (DT_ <= 2 ? 8 : 1)); break;                                                              \
    case 4: LC_DV_F32(DT_, (DT_ <= 2 ? 4 : 1)); break;                                                              \
    case 2: LC_DV_F32(DT_, (DT_ <= 4 ? 2 : 1)); break;                                                              \
    default: LC_DV_F32(DT_, 1); break;                                                                              \
  }
  switch (dt) {
    case 1: LC_DV_F32_KS(1); break;
    case 2: LC_DV_F32_KS(2); break;
    case 3: LC_DV_F32_KS(3); break;
    case 4: LC_DV_F32_KS(4); break;
    case 5: LC_DV_F32(5, 1); break;
    case 6: LC_DV_F32(6, 1); break;
    case 7: LC_DV_F32(7, 1); break;
    default: LC_DV_F32(8, 1); break;
  }
#undef LC_DV_F32_KS
#undef LC_DV_F32
  if (split_qt > 0) {
    const size_t n = static_cast<size_t>(bh) * S * D;
    const size_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
    hipLaunchKernelGGL(attn_dv_split_combine_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       split_ws, v, n, nsplit, lr);
  }
  return hipGetLastError();
}

hipError_t mseLossF32(const float* out, const float* target, size_t n, float norm, float* loss, hipStream_t stream,
                      float* partials, unsigned* counter) {
  if (n == 0) {
    return hipErrorInvalidValue;
  }
  // 16384 elements per workgroup, at most kMseLossMaxBlocks of them (one
  // workgroup without the scratch).
  size_t blocks = (n + 16383) / 16384;
  if (blocks > static_cast<size_t>(kMseLossMaxBlocks)) {
    blocks = kMseLossMaxBlocks;
  }
  if (partials == nullptr || counter == nullptr) {
    blocks = 1;
  }
  const size_t chunk = (n + blocks - 1) / blocks;
  hipLaunchKernelGGL(mse_loss_kernel, dim3(static_cast<unsigned>(blocks)), dim3(1024), 0, stream, out, target, n,
                     chunk, norm, loss, partials, counter);
  return hipGetLastError();
}

bool vitQkvAttentionFits(int T_, int E, int H) {
  return H > 0 && E % H == 0 && E / H == 64 && T_ > 0 && T_ <= 224 && E % 64 == 0 &&
         static_cast<long long>(T_) * E * 2 < (1LL << 31) && 3LL * E * E * 2 < (1LL << 31);
}

hipError_t vitQkvAttention(const uint16_t* tokens, const uint16_t* Wqkv_t, uint16_t* out_heads_concat, int B,
                           int T_, int E, int H, Half t, hipStream_t stream) {
  if (B <= 0 || !vitQkvAttentionFits(T_, E, H)) {
    return hipErrorInvalidValue;
  }
  const float scale = 1.0f / sqrtf(64.0f);
  // Two workgroups per (image, head) once there are two query blocks.
  const int nparts = T_ > 32 ? 2 : 1;
  const dim3 grid(B * H * nparts);
  // XCD blocks: tb images x th heads per XCD, tb | B, th | H, 8 blocks;
  // per XCD the L2 misses the tokens of tb images (T rows) and the weights
  // of th heads (192 rows), so minimise tb * T + th * 192.
  int tb = 0;
  int th = 0;
  if ((B * H) % 8 == 0) {
    long long best = -1;
    for (int cb = 1; cb <= B; ++cb) {
      if (B % cb != 0 || (B * H / 8) % cb != 0) {
        continue;
      }
      const int ch = B * H / 8 / cb;
      if (H % ch != 0) {
        continue;
      }
      const long long cost = static_cast<long long>(cb) * T_ + 192LL * ch;
      if (best < 0 || cost < best) {
        best = cost;
        tb = cb;
        th = ch;
      }
    }
  }
  if (t == Half::kBF16) {
    hipLaunchKernelGGL((vit_qkv_attn_kernel<BF16>), grid, dim3(512), 0, stream, tokens, Wqkv_t, out_heads_concat,
                       T_, E, H, nparts, tb, th, scale);
  } else {
    hipLaunchKernelGGL((vit_qkv_attn_kernel<F16>), grid, dim3(512), 0, stream, tokens, Wqkv_t, out_heads_concat, T_,
                       E, H, nparts, tb, th, scale);
  }
  return hipGetLastError();
}

hipError_t attentionHalf(const uint16_t* q, const uint16_t* k, const uint16_t* vt, float* out_f32,
                         uint16_t* out_heads_concat, int heads, int bh, int S, int S_pad, int D, bool causal, Half t,
                         hipStream_t stream) {
  // The K / V^T copies use 32-bit byte offsets inside one head.
  if (S <= 0 || bh <= 0 || S_pad % 128 != 0 || S_pad < S || (D != 64 && D != 128) ||
      static_cast<long long>(S_pad) * D * 2 >= (1LL << 31)) {
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
