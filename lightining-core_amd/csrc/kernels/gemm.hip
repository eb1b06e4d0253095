// gemm.hip -- MFMA GEMMs for gfx950.
//
//  * gemm_f32_kernel: fp32 in / fp32 out on v_mfma_f32_32x32x2_f32 (true fp32
//    matrix cores, no bf16x3 emulation).  64x64 block tile, BK = 16, four
//    waves in 2x2, each wave one 32x32 tile with two independent accumulator
//    chains.  LDS double buffer fed from registers; any M/N/K (edge loads are
//    zero-filled, edge stores masked).
//  * gemm_half_tn_kernel: bf16 / fp16 MFMA (v_mfma_f32_32x32x16_*), fp32
//    accumulate.  Both operands K-contiguous ("TN": C = A . Bt^T), which makes
//    every MFMA operand fetch one 16-byte LDS read.  Callers lay B out
//    transposed once at upload (the conversion pass writes it that way).
//    The A-tile loader and the epilogue are policies, so the same main loop
//    serves the plain GEMM, the implicit-GEMM patch-embed convolution and the
//    QKV projection that writes head-major Q/K and transposed V.
#include "../kernels.hpp"
#include "kcommon.hpp"

namespace lchip::k {

// ---------------------------------------------------------------------------
// fp32
// ---------------------------------------------------------------------------
constexpr int kF32BM = 64;
constexpr int kF32BN = 64;
constexpr int kF32BK = 16;

struct EpiStoreF32 {
  float* C;
  int ldc;
  __device__ __forceinline__ void operator()(int m, int n, float v) const { C[static_cast<size_t>(m) * ldc + n] = v; }
};

struct EpiConvNchwF32 {
  float* out;
  const float* bias;
  int relu;
  int oc;
  int ohw;
  __device__ __forceinline__ void operator()(int m, int n, float v) const {
    if (bias != nullptr) {
      v += bias[n];
    }
    if (relu && v < 0.0f) {
      v = 0.0f;
    }
    const int img = m / ohw;
    const int pix = m - img * ohw;
    out[(static_cast<size_t>(img) * oc + n) * ohw + pix] = v;
  }
};

// B is [K, N] (ldb) when !TRANS_B, else stored as Bt [N, K] (ldb).
template <bool VEC_A, bool VEC_B, bool TRANS_B, typename Epi>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                       int M, int N, int K, int lda, int ldb, Epi epi) {
  __shared__ float As[2][kF32BK][kF32BM + 4];
  __shared__ float Bs[2][kF32BK][kF32BN + 4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 32;
  const int wn = (wave & 1) * 32;
  const int bm = blockIdx.y * kF32BM;
  const int bn = blockIdx.x * kF32BN;

  // A: 64 rows x 16 k; thread -> row tid/4, k (tid%4)*4 .. +3.
  const int a_row = tid >> 2;
  const int a_k = (tid & 3) * 4;
  // B: 16 k x 64 n; thread -> k tid/16, n (tid%16)*4 .. +3 (!TRANS_B), or
  //    Bt: 64 n x 16 k; thread -> n tid/4, k (tid%4)*4 .. +3 (TRANS_B).
  const int b_k = TRANS_B ? (tid & 3) * 4 : (tid >> 4);
  const int b_n = TRANS_B ? (tid >> 2) : (tid & 15) * 4;

  float ra[4];
  float rb[4];
  auto load = [&](int k0) {
    const int gr = bm + a_row;
    const int gk = k0 + a_k;
    if (VEC_A && gr < M && gk + 3 < K) {
      const float4 t = *reinterpret_cast<const float4*>(A + static_cast<size_t>(gr) * lda + gk);
      ra[0] = t.x;
      ra[1] = t.y;
      ra[2] = t.z;
      ra[3] = t.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ra[j] = (gr < M && gk + j < K) ? A[static_cast<size_t>(gr) * lda + gk + j] : 0.0f;
      }
    }
    if constexpr (TRANS_B) {
      const int gn = bn + b_n;
      const int gkb = k0 + b_k;
      if (VEC_B && gn < N && gkb + 3 < K) {
        const float4 t = *reinterpret_cast<const float4*>(B + static_cast<size_t>(gn) * ldb + gkb);
        rb[0] = t.x;
        rb[1] = t.y;
        rb[2] = t.z;
        rb[3] = t.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          rb[j] = (gn < N && gkb + j < K) ? B[static_cast<size_t>(gn) * ldb + gkb + j] : 0.0f;
        }
      }
    } else {
      const int gkb = k0 + b_k;
      const int gn = bn + b_n;
      if (VEC_B && gkb < K && gn + 3 < N) {
        const float4 t = *reinterpret_cast<const float4*>(B + static_cast<size_t>(gkb) * ldb + gn);
        rb[0] = t.x;
        rb[1] = t.y;
        rb[2] = t.z;
        rb[3] = t.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          rb[j] = (gkb < K && gn + j < N) ? B[static_cast<size_t>(gkb) * ldb + gn + j] : 0.0f;
        }
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      As[buf][a_k + j][a_row] = ra[j];
    }
    if constexpr (TRANS_B) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Bs[buf][b_k + j][b_n] = rb[j];
      }
    } else {
      *reinterpret_cast<float4*>(&Bs[buf][b_k][b_n]) = make_float4(rb[0], rb[1], rb[2], rb[3]);
    }
  };

  floatx16 acc0 = zero16();
  floatx16 acc1 = zero16();
  load(0);
  store(0);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < K; k0 += kF32BK) {
    const bool more = k0 + kF32BK < K;
    if (more) {
      load(k0 + kF32BK);
    }
#pragma unroll
    for (int kk = 0; kk < kF32BK; kk += 4) {
      const float a0 = As[buf][kk + (lane >> 5)][wm + (lane & 31)];
      const float b0 = Bs[buf][kk + (lane >> 5)][wn + (lane & 31)];
      const float a1 = As[buf][kk + 2 + (lane >> 5)][wm + (lane & 31)];
      const float b1 = Bs[buf][kk + 2 + (lane >> 5)][wn + (lane & 31)];
      acc0 = mfma32x32x2f32(a0, b0, acc0);
      acc1 = mfma32x32x2f32(a1, b1, acc1);
    }
    if (more) {
      store(buf ^ 1);
    }
    __syncthreads();
    buf ^= 1;
  }

  const int n = bn + wn + (lane & 31);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = bm + wm + acc_row(i, lane);
    if (m < M && n < N) {
      epi(m, n, acc0[i] + acc1[i]);
    }
  }
}

template <bool TRANS_B, typename Epi>
static hipError_t launch_gemm_f32(const float* A, const float* B, int M, int N, int K, int lda, int ldb, Epi epi,
                                  hipStream_t stream) {
  const dim3 grid((N + kF32BN - 1) / kF32BN, (M + kF32BM - 1) / kF32BM);
  const bool va = (lda % 4 == 0) && (reinterpret_cast<uintptr_t>(A) % 16 == 0);
  const bool vb = (ldb % 4 == 0) && (reinterpret_cast<uintptr_t>(B) % 16 == 0);
  if (va && vb) {
    hipLaunchKernelGGL((gemm_f32_kernel<true, true, TRANS_B, Epi>), grid, dim3(256), 0, stream, A, B, M, N, K, lda,
                       ldb, epi);
  } else if (va) {
    hipLaunchKernelGGL((gemm_f32_kernel<true, false, TRANS_B, Epi>), grid, dim3(256), 0, stream, A, B, M, N, K, lda,
                       ldb, epi);
  } else if (vb) {
    hipLaunchKernelGGL((gemm_f32_kernel<false, true, TRANS_B, Epi>), grid, dim3(256), 0, stream, A, B, M, N, K, lda,
                       ldb, epi);
  } else {
    hipLaunchKernelGGL((gemm_f32_kernel<false, false, TRANS_B, Epi>), grid, dim3(256), 0, stream, A, B, M, N, K,
                       lda, ldb, epi);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// 16-bit TN GEMM
// ---------------------------------------------------------------------------

// A loaders: return the 16-byte chunk of A at (row, k .. k+7).
struct LoadRowMajor {
  const uint16_t* A;
  int lda;
  __device__ __forceinline__ u32x4 operator()(int row, int k) const {
    return *reinterpret_cast<const u32x4*>(A + static_cast<size_t>(row) * lda + k);
  }
};

// Implicit im2col of a patch-embed convolution (kernel = stride = P, pad 0):
// row = b*T + ty*gw + tx, k = (c*P + ky)*P + kx; 8 consecutive k are 8
// consecutive pixels of one image row.  Rows >= M read as zeros.
struct LoadPatch {
  const uint16_t* x;
  int M, C, H, W, P, T, gw;
  __device__ __forceinline__ u32x4 operator()(int row, int k) const {
    if (row >= M) {
      return u32x4{0u, 0u, 0u, 0u};
    }
    const int b = row / T;
    const int t = row - b * T;
    const int ty = t / gw;
    const int tx = t - ty * gw;
    const int pp = P * P;
    const int c = k / pp;
    const int r = k - c * pp;
    const int ky = r / P;
    const int kx = r - ky * P;
    const size_t off = ((static_cast<size_t>(b) * C + c) * H + (ty * P + ky)) * W + (tx * P + kx);
    return *reinterpret_cast<const u32x4*>(x + off);
  }
};

struct EpiF32 {
  float* C;
  int ldc;
  __device__ __forceinline__ void operator()(int m, int n, float v) const { C[static_cast<size_t>(m) * ldc + n] = v; }
};

template <typename T>
struct EpiHalf {
  uint16_t* C;
  int ldc;
  int relu;
  __device__ __forceinline__ void operator()(int m, int n, float v) const {
    if (relu && v < 0.0f) {
      v = 0.0f;
    }
    C[static_cast<size_t>(m) * ldc + n] = to_half_bits<T>(v);
  }
};

// qkv[m = b*T + t, n = which*E + h*Dh + d] -> Q/K [b*H + h, t, d], Vt [b*H + h, d, t].
template <typename T>
struct EpiQKV {
  uint16_t* q;
  uint16_t* k;
  uint16_t* vt;
  int T_;
  int E;
  int H;
  int Dh;
  int S_pad;
  __device__ __forceinline__ void operator()(int m, int n, float v) const {
    const int b = m / T_;
    const int t = m - b * T_;
    const int which = n / E;
    const int r = n - which * E;
    const int h = r / Dh;
    const int d = r - h * Dh;
    const size_t head = static_cast<size_t>(b) * H + h;
    const uint16_t bits = to_half_bits<T>(v);
    if (which == 0) {
      q[(head * S_pad + t) * Dh + d] = bits;
    } else if (which == 1) {
      k[(head * S_pad + t) * Dh + d] = bits;
    } else {
      vt[(head * Dh + d) * S_pad + t] = bits;
    }
  }
};

template <typename T, int BM, int BN, int BK, int WM, int WN, typename LoadA, typename Epi>
__global__ __launch_bounds__(WM* WN * 64) void gemm_half_tn_kernel(LoadA load_a, const uint16_t* __restrict__ Bt,
                                                                    int M, int N, int K, int ldb, int tiles_n,
                                                                    Epi epi) {
  constexpr int NT = WM * WN * 64;
  constexpr int LDK = BK + 8;  // LDS row stride (elements): +16 B breaks bank aliasing
  constexpr int TM = BM / WM / 32;
  constexpr int TN = BN / WN / 32;
  constexpr int KCH = BK / 8;  // 16-byte chunks per tile row
  constexpr int CA = BM * KCH / NT;
  constexpr int CB = BN * KCH / NT;
  static_assert(CA * NT == BM * KCH && CB * NT == BN * KCH, "tile / thread mismatch");

  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave / WN) * (BM / WM);
  const int wn = (wave % WN) * (BN / WN);

  // Block -> tile mapping.  The dispatcher hands workgroup i to XCD i % 8;
  // remap so each XCD receives a contiguous run of the grouped tile order
  // (tiles that share A row panels and B column panels), which then hit in
  // that XCD's own L2.  Grouped order: 8 tile-rows share their B panels.
  constexpr int GROUP = 8;
  const int tiles_m = (M + BM - 1) / BM;
  const int nwg = gridDim.x;
  const int full = nwg & ~7;
  int pid = blockIdx.x;
  if (pid < full) {
    pid = (pid & 7) * (full >> 3) + (pid >> 3);
  }
  const int group_size = GROUP * tiles_n;
  const int group = pid / group_size;
  const int first_m = group * GROUP;
  const int gm = min(tiles_m - first_m, GROUP);
  const int in_group = pid - group * group_size;
  const int tile_m = first_m + in_group % gm;
  const int tile_n = in_group / gm;
  const int bm = tile_m * BM;
  const int bn = tile_n * BN;

  u32x4 ra[CA];
  u32x4 rb[CB];
  auto load = [&](int k0) {
#pragma unroll
    for (int c = 0; c < CA; ++c) {
      const int idx = c * NT + tid;
      const int row = idx / KCH;
      const int col = (idx - row * KCH) * 8;
      ra[c] = load_a(bm + row, k0 + col);
    }
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const int idx = c * NT + tid;
      const int row = idx / KCH;
      const int col = (idx - row * KCH) * 8;
      rb[c] = *reinterpret_cast<const u32x4*>(Bt + static_cast<size_t>(bn + row) * ldb + k0 + col);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int c = 0; c < CA; ++c) {
      const int idx = c * NT + tid;
      const int row = idx / KCH;
      const int col = (idx - row * KCH) * 8;
      *reinterpret_cast<u32x4*>(&As[buf][row * LDK + col]) = ra[c];
    }
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const int idx = c * NT + tid;
      const int row = idx / KCH;
      const int col = (idx - row * KCH) * 8;
      *reinterpret_cast<u32x4*>(&Bs[buf][row * LDK + col]) = rb[c];
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      acc[i][j] = zero16();
    }
  }

  load(0);
  store(0);
  __syncthreads();
  int buf = 0;
  const int lrow = lane & 31;
  const int lk = 8 * (lane >> 5);
  for (int k0 = 0; k0 < K; k0 += BK) {
    const bool more = k0 + BK < K;
    if (more) {
      load(k0 + BK);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      u32x4 af[TM];
      u32x4 bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        af[i] = *reinterpret_cast<const u32x4*>(&As[buf][(wm + i * 32 + lrow) * LDK + kk + lk]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        bf[j] = *reinterpret_cast<const u32x4*>(&Bs[buf][(wn + j * 32 + lrow) * LDK + kk + lk]);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          acc[i][j] = mfma32x32x16<T>(af[i], bf[j], acc[i][j]);
        }
      }
    }
    if (more) {
      store(buf ^ 1);
    }
    __syncthreads();
    buf ^= 1;
  }

#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = bn + wn + j * 32 + lrow;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = bm + wm + i * 32 + acc_row(r, lane);
        if (m < M && n < N) {
          epi(m, n, acc[i][j][r]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny 16-bit GEMM (M <= 16): HBM-bound on streaming Bt once.  Each
// workgroup owns NT 16-column tiles; its 4 waves take interleaved 32-wide
// k-steps (so together they read 256 contiguous bytes of each Bt row per
// round) with v_mfma_f32_16x16x32_*, and the 4 partial tiles are summed
// through LDS.  A (16 rows) is re-read per tile from L2.
//   16x16x32 layout: A[m = l%16][k = 8(l/16)+j], B[k = 8(l/16)+j][n = l%16],
//   D[m = 4(l/16) + i][n = l%16], i = 0..3.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ floatx4 mfma16x16x32(u32x4 a, u32x4 b, floatx4 c);
template <>
__device__ __forceinline__ floatx4 mfma16x16x32<BF16>(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}
template <>
__device__ __forceinline__ floatx4 mfma16x16x32<F16>(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

template <typename T, int NT>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(const uint16_t* __restrict__ A,
                                                          const uint16_t* __restrict__ Bt, float* __restrict__ C,
                                                          int M, int N, int K, int lda, int ldb, int ldc) {
  __shared__ floatx4 red[4][NT][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16 * NT;
  const int r16 = lane & 15;
  const int kofs = 8 * (lane >> 4);
  const uint16_t* arow = A + static_cast<size_t>(r16) * lda + kofs;
  const uint16_t* brow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    brow[t] = Bt + static_cast<size_t>(n0 + t * 16 + r16) * ldb + kofs;
  }
  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const int steps = K / 32;
  int s = wave;
  for (; s + 12 < steps; s += 16) {
    u32x4 a[4];
    u32x4 b[4][NT];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[u] = *reinterpret_cast<const u32x4*>(arow + (s + 4 * u) * 32);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        b[u][t] = *reinterpret_cast<const u32x4*>(brow[t] + (s + 4 * u) * 32);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        acc[t] = mfma16x16x32<T>(a[u], b[u][t], acc[t]);
      }
    }
  }
  for (; s < steps; s += 4) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(arow + s * 32);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      acc[t] = mfma16x16x32<T>(a, *reinterpret_cast<const u32x4*>(brow[t] + s * 32), acc[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    red[wave][t][lane] = acc[t];
  }
  __syncthreads();
  if (wave < NT) {
    const int t = wave;
    floatx4 v = red[0][t][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const floatx4 o = red[w][t][lane];
      v[0] += o[0];
      v[1] += o[1];
      v[2] += o[2];
      v[3] += o[3];
    }
    const int n = n0 + t * 16 + r16;
    if (n < N) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * (lane >> 4) + i;
        if (m < M) {
          C[static_cast<size_t>(m) * ldc + n] = v[i];
        }
      }
    }
  }
}

constexpr int kHBK = 64;

// Tile configurations (block tile BM x BN, waves WM x WN):
//   big   256x256, 8 waves (2 x 4, 128x64 each), 147 KB LDS double buffer
//   mid   128x128, 4 waves (2 x 2, 64x64 each)
//   small  64x64,  4 waves (2 x 2, 32x32 each)
// The largest tile that still gives at least one workgroup per CU is used.
enum class HalfTile { kBig, kMid, kSmall };

inline int tiles_for(int M, int N, int b) { return ((M + b - 1) / b) * ((N + b - 1) / b); }

inline HalfTile pick_half_tile(int M, int N) {
  constexpr int kCUs = 256;
  if (tiles_for(M, N, 256) >= kCUs) {
    return HalfTile::kBig;
  }
  if (tiles_for(M, N, 128) >= kCUs) {
    return HalfTile::kMid;
  }
  return HalfTile::kSmall;
}

template <typename T, int BM, int BN, int WM, int WN, typename LoadA, typename Epi>
static hipError_t launch_gemm_half_cfg(LoadA load_a, const uint16_t* Bt, int M, int N, int K, int ldb, Epi epi,
                                       hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_half_tn_kernel<T, BM, BN, kHBK, WM, WN, LoadA, Epi>), dim3(tiles_m * tiles_n),
                     dim3(WM * WN * 64), 0, stream, load_a, Bt, M, N, K, ldb, tiles_n, epi);
  return hipGetLastError();
}

template <typename T, typename LoadA, typename Epi>
static hipError_t launch_gemm_half(LoadA load_a, const uint16_t* Bt, int M, int N, int K, int ldb, Epi epi,
                                   hipStream_t stream) {
  switch (pick_half_tile(M, N)) {
    case HalfTile::kBig:
      return launch_gemm_half_cfg<T, 256, 256, 2, 4>(load_a, Bt, M, N, K, ldb, epi, stream);
    case HalfTile::kMid:
      return launch_gemm_half_cfg<T, 128, 128, 2, 2>(load_a, Bt, M, N, K, ldb, epi, stream);
    case HalfTile::kSmall:
    default:
      return launch_gemm_half_cfg<T, 64, 64, 2, 2>(load_a, Bt, M, N, K, ldb, epi, stream);
  }
}

}  // namespace lchip::k

namespace lchip::kern {

using namespace lchip::k;

hipError_t gemmF32(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                   hipStream_t stream) {
  return launch_gemm_f32<false>(A, B, M, N, K, lda, ldb, EpiStoreF32{C, ldc}, stream);
}

hipError_t gemmF32ConvNchw(const float* cols, const float* Wt, float* out, int M, int N, int K, const float* bias,
                           int relu, int ohw, hipStream_t stream) {
  return launch_gemm_f32<true>(cols, Wt, M, N, K, K, K, EpiConvNchwF32{out, bias, relu, N, ohw}, stream);
}

hipError_t gemmHalfTN(const uint16_t* A, const uint16_t* Bt, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                      Half t, hipStream_t stream) {
  if (K % kHBK != 0) {
    return hipErrorInvalidValue;
  }
  if (M <= 16) {
    // Bt must be readable up to roundup(N, 32) rows (callers pad to 256).
    constexpr int NT = 2;
    const dim3 grid((N + 16 * NT - 1) / (16 * NT));
    if (t == Half::kBF16) {
      hipLaunchKernelGGL((gemm_skinny_kernel<BF16, NT>), grid, dim3(256), 0, stream, A, Bt, C, M, N, K, lda, ldb, ldc);
    } else {
      hipLaunchKernelGGL((gemm_skinny_kernel<F16, NT>), grid, dim3(256), 0, stream, A, Bt, C, M, N, K, lda, ldb, ldc);
    }
    return hipGetLastError();
  }
  const LoadRowMajor la{A, lda};
  if (t == Half::kBF16) {
    return launch_gemm_half<BF16>(la, Bt, M, N, K, ldb, EpiF32{C, ldc}, stream);
  }
  return launch_gemm_half<F16>(la, Bt, M, N, K, ldb, EpiF32{C, ldc}, stream);
}

hipError_t gemmHalfTNHalfOut(const uint16_t* A, const uint16_t* Bt, uint16_t* C, int M, int N, int K, int lda,
                             int ldb, int ldc, int relu, Half t, hipStream_t stream) {
  if (K % kHBK != 0) {
    return hipErrorInvalidValue;
  }
  const LoadRowMajor la{A, lda};
  if (t == Half::kBF16) {
    return launch_gemm_half<BF16>(la, Bt, M, N, K, ldb, EpiHalf<BF16>{C, ldc, relu}, stream);
  }
  return launch_gemm_half<F16>(la, Bt, M, N, K, ldb, EpiHalf<F16>{C, ldc, relu}, stream);
}

hipError_t patchEmbedGemm(const uint16_t* x, const uint16_t* Wt, uint16_t* tokens, int B, int C, int H, int W, int P,
                          int E, Half t, hipStream_t stream) {
  const int gh = H / P;
  const int gw = W / P;
  const int T_ = gh * gw;
  const int M = B * T_;
  const int K = C * P * P;
  if (P % 8 != 0 || K % kHBK != 0 || W % 8 != 0) {
    return hipErrorInvalidValue;
  }
  const LoadPatch la{x, M, C, H, W, P, T_, gw};
  if (t == Half::kBF16) {
    return launch_gemm_half<BF16>(la, Wt, M, E, K, K, EpiHalf<BF16>{tokens, E, 1}, stream);
  }
  return launch_gemm_half<F16>(la, Wt, M, E, K, K, EpiHalf<F16>{tokens, E, 1}, stream);
}

hipError_t qkvProjectGemm(const uint16_t* tokens, const uint16_t* Wqkv_t, uint16_t* q, uint16_t* k, uint16_t* vt,
                          int B, int T_, int E, int H, int S_pad, Half t, hipStream_t stream) {
  const int M = B * T_;
  if (E % kHBK != 0 || E % H != 0) {
    return hipErrorInvalidValue;
  }
  const LoadRowMajor la{tokens, E};
  const int Dh = E / H;
  if (t == Half::kBF16) {
    return launch_gemm_half<BF16>(la, Wqkv_t, M, 3 * E, E, E, EpiQKV<BF16>{q, k, vt, T_, E, H, Dh, S_pad}, stream);
  }
  return launch_gemm_half<F16>(la, Wqkv_t, M, 3 * E, E, E, EpiQKV<F16>{q, k, vt, T_, E, H, Dh, S_pad}, stream);
}

}  // namespace lchip::kern
