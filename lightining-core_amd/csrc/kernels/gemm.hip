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
#include <stdlib.h>

#include <string>
#include <type_traits>

#include "../kernels.hpp"
#include "kcommon.hpp"

namespace lchip::k {

using kern::StreamKSync;

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
  int vec4 = 0;  // C is 16-byte aligned and ldc % 4 == 0 (store4 may use one 16-byte store)
  __device__ __forceinline__ void operator()(int m, int n, float v) const { C[static_cast<size_t>(m) * ldc + n] = v; }
  // C[m][n .. n + 3] = v[0 .. 3] (n a multiple of 4), columns >= N dropped.
  __device__ __forceinline__ void store4(int m, int n, int N, floatx4 v) const {
    float* p = C + static_cast<size_t>(m) * ldc + n;
    if (vec4 && n + 3 < N) {
      *reinterpret_cast<floatx4*>(p) = v;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (n + r < N) {
          p[r] = v[r];
        }
      }
    }
  }
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
  // A whole 32x32 accumulator of one lane: column n (one head and d for the
  // lane), rows mbase + 8g + 4*(lane/32) + i, i < 4, for g < 4.  Each group of
  // 4 rows lies in one image when T_ % 4 == 0 (the caller checks), so its
  // token index comes from one division and its 4 V^T values are one 8-byte
  // store; Q and K rows stay 2-byte stores, 32 lanes to 64 contiguous bytes.
  static constexpr bool kAccStore = true;
  __device__ __forceinline__ void store_acc(int mbase, int n, const floatx16& acc, int lane, int M, int N) const {
    if (n >= N) {
      return;
    }
    const int which = n / E;
    const int r = n - which * E;
    const int h = r / Dh;
    const int d = r - h * Dh;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int m0 = mbase + 8 * g + 4 * (lane >> 5);
      if (m0 >= M) {
        continue;
      }
      const int b = m0 / T_;
      const int t0 = m0 - b * T_;
      const size_t head = static_cast<size_t>(b) * H + h;
      if (which == 2) {
        u32x2 w;
        w[0] = pack2<T>(acc[4 * g], acc[4 * g + 1]);
        w[1] = pack2<T>(acc[4 * g + 2], acc[4 * g + 3]);
        *reinterpret_cast<u32x2*>(vt + (head * Dh + d) * S_pad + t0) = w;
      } else {
        uint16_t* dst = (which == 0 ? q : k) + (head * S_pad + t0) * Dh + d;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dst[i * Dh] = to_half_bits<T>(acc[4 * g + i]);
        }
      }
    }
  }
};

// Whether an epilogue stores whole accumulators (store_acc) instead of
// single elements.
template <typename E, typename = void>
struct AccStore {
  static constexpr bool value = false;
};
template <typename E>
struct AccStore<E, decltype(void(E::kAccStore))> {
  static constexpr bool value = E::kAccStore;
};

template <typename T, int BM, int BN, int BK, int WM, int WN, int STORE_AT, typename LoadA, typename Epi>
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
      // The next stage goes to the other LDS buffer half-way through this
      // stage's MFMAs, so the store (and its wait on the global loads)
      // overlaps matrix work instead of following it.
      if (kk == STORE_AT && more) {
        store(buf ^ 1);
      }
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
    if (STORE_AT >= BK && more) {
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
// Skinny 16-bit GEMM (M <= 16): HBM-bound on streaming Bt once.
//
// A workgroup owns NR = 16*NT rows of Bt (columns of C) and one of KS
// contiguous k-ranges (split-K, grid.y).  Rows are staged in LDS by
// LDS-DMA in k-blocks of 256: each copy instruction reads 1 KB of global
// memory contiguously (two rows x 512 bytes), which is what lets HBM stream
// near its peak (the MFMA-layout loads of 16 rows x 64 bytes stop near 5
// TB/s).  The 16 rows of A ride along in the same stages.  Within a row the
// 16-byte chunks are XOR-swizzled by (row & 15), so the 16 rows of an MFMA
// fragment read sit in distinct LDS banks.  Two stages: block b+1 loads
// while block b is multiplied (v_mfma_f32_16x16x32, the W waves taking the
// block's 32-wide k-steps in turn).  With KS == 1 workgroup ct walks its
// k-blocks starting at block (5 * ct) % nkb and wrapping around: workgroups
// that run together then read different 512-byte column slabs of their rows
// instead of the same slab 16 KB apart in every row, which spreads their
// reads over the HBM channels (16x8192x8192: 23.9 -> 21.3 us at 128
// workgroups).  The W partial tiles are summed through
// LDS (over the stages, all reads done).  With KS > 1 each workgroup stores
// its partial to the workspace with device-scope stores, waits for them,
// and bumps its column tile's counter; the one that brings it to KS sums the
// KS partials in k order (deterministic), writes C and resets the counter to
// zero for the next launch.  No workgroup ever waits for another.
//   16x16x32 layout: A[m = l%16][k = 8(l/16)+j], B[k = 8(l/16)+j][n = l%16],
//   D[m = 4(l/16) + i][n = l%16], i = 0..3 (mfma16x16x32, kcommon.hpp).
// ---------------------------------------------------------------------------

constexpr int kSkinnyNT = 4;     // 16-column tiles per workgroup
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyStages = 2;
constexpr int kSkinnyKB = 256;   // k per stage

template <typename T, int NT, int W, int S>
__global__ __launch_bounds__(W * 64) void gemm_skinny_kernel(const uint16_t* __restrict__ A,
                                                              const uint16_t* __restrict__ Bt,
                                                              float* __restrict__ C, int M, int N, int K, int lda,
                                                              int ldb, int ldc, float* __restrict__ part,
                                                              int* __restrict__ counters) {
  constexpr int NR = 16 * NT;              // Bt rows per workgroup
  constexpr int ROWS = NR + 16;            // + the 16 rows of A
  constexpr int KB = kSkinnyKB;
  constexpr int STAGE = ROWS * KB;         // elements per stage
  constexpr int PAIRS = ROWS / 2 / W;      // copy instructions per wave per stage
  static_assert((ROWS / 2) % W == 0 && (NR / 2) % W == 0, "row pairs per wave");
  static_assert(W >= NT, "one wave per column tile in the final sum");
  static_assert(W * NT * 1024 + 16 <= S * STAGE * 2, "partials and flag fit over the stages");
  __shared__ __attribute__((aligned(16))) uint16_t sm[S * STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ct = blockIdx.x;
  const int ks = blockIdx.y;
  const int KS = gridDim.y;
  const int n0 = ct * NR;
  const uint32_t lds0 = lds_addr(sm);
  const int nkb = (K + KB - 1) / KB;
  const int per = (nkb + KS - 1) / KS;
  const int kb0 = min(nkb, ks * per);
  const int kb1 = min(nkb, kb0 + per);
  // Copy of k-block kb into stage st: instruction i of wave w fills rows
  // 2p, 2p+1 (p = w + W*i; Bt rows first, then A's); lane l reads 16 bytes of
  // row 2p + l/32 at logical chunk (l%32) ^ (row & 15), which lands at
  // physical chunk l%32.  Chunks past K are not read.
  auto issue = [&](int kb, int st) {
    const int k0 = kb * KB;
    const int valid = min(KB, K - k0) / 8;
#pragma unroll
    for (int i = 0; i < PAIRS; ++i) {
      const int r0 = 2 * (wave + W * i);
      const bool is_b = i < NR / 2 / W;
      const uint16_t* src = is_b ? Bt + static_cast<size_t>(n0 + r0) * ldb : A + static_cast<size_t>(r0 - NR) * lda;
      const int ld = is_b ? ldb : lda;
      const int rr = r0 + (lane >> 5);
      const int chunk = (lane & 31) ^ (rr & 15);
      if (chunk < valid) {
        load_lds16_sbase(static_cast<uint32_t>(((lane >> 5) * ld + k0 + chunk * 8) * 2), src,
                         lds0 + 2u * static_cast<uint32_t>(st * STAGE + r0 * KB));
      }
    }
  };
  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const int r16 = lane & 15;
  const int cg = lane >> 4;
  // The i-th block this workgroup multiplies (i < nb): its range rotated by
  // rot when unsplit, in k order otherwise.
  const int nb = kb1 - kb0;
  const int rot = (KS == 1 && nb > 0) ? (5 * ct) % nb : 0;
  auto block = [&](int i) {
    const int q = i + rot;
    return kb0 + (q >= nb ? q - nb : q);
  };
#pragma unroll
  for (int p = 0; p < S - 1; ++p) {
    if (p < nb) {
      issue(block(p), p);
    }
  }
  for (int sl = 0; sl < nb; ++sl) {
    if (sl + S - 1 < nb) {
      issue(block(sl + S - 1), (sl + S - 1) % S);
      wait_vmcnt<(S - 1) * PAIRS>();  // this wave's copies of block sl have landed
    } else {
      wait_vmcnt<0>();
    }
    stage_barrier();  // everyone's have
    const uint16_t* st = sm + (sl % S) * STAGE;
    const int steps = min(KB, K - block(sl) * KB) / 32;
    for (int s = wave; s < steps; s += W) {
      const int ch = 4 * s + cg;  // logical 16-byte chunk of this lane's 8 k
      const u32x4 a = *reinterpret_cast<const u32x4*>(st + (NR + r16) * KB + ((ch ^ r16) << 3));
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int r = t * 16 + r16;
        const u32x4 b = *reinterpret_cast<const u32x4*>(st + r * KB + ((ch ^ (r & 15)) << 3));
        acc[t] = mfma16x16x32<T>(a, b, acc[t]);
      }
    }
    stage_barrier();  // the stage is refilled next
  }
  floatx4* red = reinterpret_cast<floatx4*>(sm);  // [W][NT][64]
  int* last = reinterpret_cast<int*>(sm + W * NT * 512);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    red[(wave * NT + t) * 64 + lane] = acc[t];
  }
  __syncthreads();
  floatx4 v = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  if (wave < NT) {
    v = red[wave * 64 + lane];
#pragma unroll
    for (int w = 1; w < W; ++w) {
      const floatx4 o = red[(w * NT + wave) * 64 + lane];
      v[0] += o[0];
      v[1] += o[1];
      v[2] += o[2];
      v[3] += o[3];
    }
  }
  auto store_c = [&](const floatx4& x) {
    const int n = n0 + wave * 16 + r16;
    if (n < N) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * cg + i;
        if (m < M) {
          C[static_cast<size_t>(m) * ldc + n] = x[i];
        }
      }
    }
  };
  if (KS == 1) {
    if (wave < NT) {
      store_c(v);
    }
    return;
  }
  // Partial of (ct, ks) at part[((ct * KS + ks) * NT + t) * 256 + i * 64 + lane].
  // Device-scope (sc1) stores and loads are coherent across the XCDs' L2s;
  // the vmcnt wait orders the stores before the counter bump.
  if (wave < NT) {
    float* mine = part + (static_cast<size_t>(ct * KS + ks) * NT + wave) * 256 + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __hip_atomic_store(mine + i * 64, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) {
    *last = __hip_atomic_fetch_add(counters + ct, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == KS - 1;
  }
  __syncthreads();
  if (*last == 0) {
    return;
  }
  if (wave < NT) {
    floatx4 x = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k2 = 0; k2 < KS; ++k2) {
      const float* theirs = part + (static_cast<size_t>(ct * KS + k2) * NT + wave) * 256 + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] += __hip_atomic_load(theirs + i * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    store_c(x);
  }
  if (threadIdx.x == 0) {
    __hip_atomic_store(counters + ct, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

constexpr int kHBK = 64;

// ---------------------------------------------------------------------------
// Large-tile 16-bit TN GEMM with direct global -> LDS loads.
//
// 256x256 block tile, BK = 64, 8 waves (2 x 4, each 128x64), two LDS stages
// of 64 KB.  global_load_lds_dwordx4 writes each lane's 16 bytes to
// LDS base + 16*lane, so one wave instruction fills 1 KB = 8 tile rows of
// 128 bytes; which global chunk a lane fetches is free, and it is chosen so
// the LDS rows are XOR-swizzled (physical chunk = logical chunk ^
// ((row >> 1) & 7)).  gfx950's LDS serves a 16-byte read for 16 lanes per
// clock (256 bytes, 64 banks); a fragment read puts 16 consecutive rows of
// one logical chunk in such a group, and with 128-byte rows even and odd rows
// land in opposite bank halves, so the swizzle only has to separate the 8
// even (and 8 odd) rows: conflict-free without padding.  No
// staging registers and no LDS store instructions: the freed registers
// double-buffer the MFMA fragments, so each k-step's LDS reads are issued
// one step ahead of its MFMAs.  Stage k+1 is loaded while stage k is
// computed; one wait + barrier per stage.  The copies use a scalar tile base
// and fixed 32-bit lane offsets (load_lds16_sbase): the host keeps
// 256 * ld * 2 bytes below 2^31.
// ---------------------------------------------------------------------------
template <typename T, int WM, int WN, typename Epi>
__global__ __launch_bounds__(WM* WN * 64) void gemm_half_tn_lds_kernel(const uint16_t* __restrict__ A,
                                                                         const uint16_t* __restrict__ Bt, int M,
                                                                         int N, int K, int lda, int ldb, int tiles_n,
                                                                         Epi epi) {
  constexpr int BM = 256, BN = 256, BK = 64;
  constexpr int NW = WM * WN;        // waves
  constexpr int LPW = 32 / NW;       // 1 KB load instructions per wave per operand
  constexpr int TM = BM / WM / 32;
  constexpr int TN = BN / WN / 32;
  constexpr int ROWB = BK * 2;      // bytes per LDS row (128)
  constexpr int STAGE = (BM + BN) * BK;  // elements per stage
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave / WN) * (BM / WM);
  const int wn = (wave % WN) * (BN / WN);

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
  const int bm = (first_m + in_group % gm) * BM;
  const int bn = (in_group / gm) * BN;

  // Load mapping: instruction i (of 32 per operand) fills tile rows 8i..8i+7;
  // wave w issues i = NW*j + w, j = 0 .. 32/NW - 1.  Lane l -> row 8i + l/8, physical
  // chunk l%8, logical chunk (l%8) ^ ((row >> 1) & 7).
  const int lrow8 = lane >> 3;
  const int pchunk = lane & 7;
  uint32_t a_off[LPW];  // byte offsets inside the tile's rows, fixed for all stages
  uint32_t b_off[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int row = 8 * (NW * j + wave) + lrow8;
    const int lchunk = pchunk ^ ((row >> 1) & 7);
    a_off[j] = static_cast<uint32_t>(row * lda + lchunk * 8) * 2u;
    b_off[j] = static_cast<uint32_t>(row * ldb + lchunk * 8) * 2u;
  }
  const uint16_t* a_tile = A + static_cast<size_t>(bm) * lda;
  const uint16_t* b_tile = Bt + static_cast<size_t>(bn) * ldb;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = lds_addr(smem);
  // Copy q of a stage: A rows for q < LPW, then B rows.
  auto issue_one = [&](int buf, int k0, int q) {
    const uint32_t base = lds0 + 2u * static_cast<uint32_t>(buf * STAGE);
    if (q < LPW) {
      load_lds16_sbase(a_off[q], a_tile + k0, base + 2u * static_cast<uint32_t>((NW * q + wave_s) * 8 * BK));
    } else {
      load_lds16_sbase(b_off[q - LPW], b_tile + k0,
                       base + 2u * static_cast<uint32_t>(BM * BK + (NW * (q - LPW) + wave_s) * 8 * BK));
    }
  };
  auto issue = [&](int buf, int k0) {
#pragma unroll
    for (int q = 0; q < 2 * LPW; ++q) {
      issue_one(buf, k0, q);
    }
  };

  // Fragment read: row r, logical chunk c -> byte r*128 + ((c ^ (r&7)) * 16).
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  auto frag = [&](const uint16_t* base, int row, int c) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + row * ROWB +
                                           ((c ^ ((row >> 1) & 7)) << 4));
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      acc[i][j] = zero16();
    }
  }

  const int nk = K / BK;
  issue(0, 0);
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0); expcnt / lgkmcnt left at their maxima
  __syncthreads();
  // Only this wave's LDS reads may be outstanding at the loop head: a pending
  // scalar load would make every LDS wait in the loop an lgkmcnt(0).
  __builtin_amdgcn_s_waitcnt(0xc07f);
  // The next stage's copies go out one after every second MFMA of this
  // stage's first two k-steps (8 copies per wave): issued in a burst they
  // queue behind the other waves' copies and hold up this wave's MFMAs;
  // spread over the whole stage the last ones land late.
  constexpr int MPS = TM * TN;                 // MFMAs per k-step
  constexpr int EVERY = 2;
  constexpr int COPIES = 2 * LPW;
  static_assert(COPIES <= 2 * MPS / EVERY, "copies fit the first two k-steps");
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    const uint16_t* As = smem + buf * STAGE;
    const uint16_t* Bs = As + BM * BK;
    u32x4 af[2][TM];
    u32x4 bf[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      af[0][i] = frag(As, wm + i * 32 + lrow, lhalf);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      bf[0][j] = frag(Bs, wn + j * 32 + lrow, lhalf);
    }
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int cur = s & 1;
      if (s + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          af[cur ^ 1][i] = frag(As, wm + i * 32 + lrow, 2 * (s + 1) + lhalf);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          bf[cur ^ 1][j] = frag(Bs, wn + j * 32 + lrow, 2 * (s + 1) + lhalf);
        }
      }
      // Keep the next step's LDS reads ahead of this step's MFMAs (the
      // scheduler would otherwise sink them next to their use and expose the
      // full LDS latency before every MFMA group).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          acc[i][j] = mfma32x32x16<T>(af[cur][i], bf[cur][j], acc[i][j]);
          const int mi = s * MPS + i * TN + j;  // MFMA index within the stage
          if (mi % EVERY == EVERY - 1 && mi / EVERY < COPIES && more) {
            __builtin_amdgcn_sched_barrier(0);
            issue_one(buf ^ 1, (kt + 1) * BK, mi / EVERY);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);  // this wave's loads of stage kt+1 have landed
    stage_barrier();                      // everyone's have; everyone is done with stage kt
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
// 16-bit TN GEMM for grids of at least two 256x256 tiles per CU: 4 waves of
// 128x128 (one per SIMD, accumulators in the AGPRs), against the 8 waves of
// 128x64 above: half the LDS fragment reads per MFMA.
//
// LDS holds a ring of four 32-deep k slices (32 KB each: 256 A rows then 256
// B rows of 64 bytes, 16-byte chunk c of row r at physical chunk
// c ^ ((r >> 2) & 3), conflict-free for the fragment reads).  During slice h
// a wave issues its 8 copies of slice h + 3 (into the slot slice h - 1 left,
// one after every fourth MFMA), reads the fragments of k-step 1 of slice h
// and then k-step 0 of slice h + 1 while its MFMAs run; at the end of slice h
// it waits for its copies of slice h + 2 and the barrier publishes them, so
// no fragment read waits on a barrier.  Past the last slice the copies
// re-load slice H - 1 into slots already retired and the reads of slot
// (h + 1) & 3 return unused data: every iteration has the same waits.
//
// The k order of each accumulator matches gemm_half_tn_lds_kernel, so the two
// give bit-identical results.  Tiles are ordered in groups of 4 tile rows per
// XCD (measured on 8192^3: 4 against 8, 2, 16 and 1: 4%, 12%, 13% and 50%
// faster).  Operands are padded to
// 256 rows and copies use 32-bit lane offsets: the host keeps 256 * ld * 2
// bytes below 2^31.
// ---------------------------------------------------------------------------
template <typename T, typename Epi>
__global__ __launch_bounds__(256) void gemm_half_tn_w4_kernel(const uint16_t* __restrict__ A,
                                                              const uint16_t* __restrict__ Bt, int M, int N, int K,
                                                              int lda, int ldb, int tiles_n, Epi epi) {
  constexpr int BM = 256, BN = 256, HK = 32;
  constexpr int ROWB = HK * 2;            // bytes per LDS row (64)
  constexpr int SLOT = (BM + BN) * HK;    // elements per slot
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * SLOT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;

  constexpr int GROUP = 4;
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
  const int bm = (first_m + in_group % gm) * BM;
  const int bn = (in_group / gm) * BN;

  // Copy instruction i (0..15 per operand per slice) fills rows 16i + lane/4,
  // physical chunk lane%4; wave w issues i = w + 4j, j = 0..3.
  const int crow = lane >> 2;
  const int pch = lane & 3;
  uint32_t a_off[4];
  uint32_t b_off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 16 * (wave + 4 * j) + crow;
    const int lch = pch ^ ((row >> 2) & 3);
    a_off[j] = static_cast<uint32_t>(row * lda + lch * 8) * 2u;
    b_off[j] = static_cast<uint32_t>(row * ldb + lch * 8) * 2u;
  }
  const uint16_t* a_tile = A + static_cast<size_t>(bm) * lda;
  const uint16_t* b_tile = Bt + static_cast<size_t>(bn) * ldb;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = lds_addr(smem);
  // Copy q (0..7) of slice h into ring slot `slot`: A rows for q < 4, then B.
  auto issue_one = [&](int h, int q, int slot) {
    const uint32_t base = lds0 + 2u * static_cast<uint32_t>((slot & 3) * SLOT);
    const int k0 = h * HK;
    if (q < 4) {
      load_lds16_sbase(a_off[q], a_tile + k0, base + static_cast<uint32_t>((wave_s + 4 * q) * 1024));
    } else {
      load_lds16_sbase(b_off[q - 4], b_tile + k0,
                       base + 2u * BM * HK + static_cast<uint32_t>((wave_s + 4 * (q - 4)) * 1024));
    }
  };

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  // Fragment f (0..7) of k-step s of slice h: A rows for f < 4, then B rows.
  auto frag = [&](int h, int s, int f) -> u32x4 {
    const char* base = reinterpret_cast<const char*>(smem + (h & 3) * SLOT);
    const int row = f < 4 ? wm + f * 32 + lrow : wn + (f - 4) * 32 + lrow;
    const int opoff = f < 4 ? 0 : 2 * BM * HK;
    const int c = 2 * s + lhalf;
    return *reinterpret_cast<const u32x4*>(base + opoff + row * ROWB + ((c ^ ((row >> 2) & 3)) << 4));
  };

  floatx16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = zero16();
    }
  }

  const int H = K / HK;
#pragma unroll
  for (int h = 0; h < 3; ++h) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      issue_one(min(h, H - 1), q, h);
    }
  }
  wait_vmcnt<8>();                     // slices 0 and 1 have landed
  __builtin_amdgcn_s_waitcnt(0xc07f);  // no scalar load pending at the loop head
  stage_barrier();
  u32x4 f0[8];
  u32x4 f1[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    f0[f] = frag(0, 0, f);
  }
  for (int h = 0; h < H; ++h) {
    const int hc = min(h + 3, H - 1);
    // k-step 0: MFMAs on f0; f1 <- k-step 1 of slice h; copies 0..3
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i >> 2][i & 3] = mfma32x32x16<T>(f0[i >> 2], f0[4 + (i & 3)], acc[i >> 2][i & 3]);
      __builtin_amdgcn_sched_barrier(0);
      if (i < 8) {
        f1[i] = frag(h, 1, i);
      }
      if ((i & 3) == 3) {
        issue_one(hc, i >> 2, h + 3);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // k-step 1: MFMAs on f1; f0 <- k-step 0 of slice h + 1; copies 4..7
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i >> 2][i & 3] = mfma32x32x16<T>(f1[i >> 2], f1[4 + (i & 3)], acc[i >> 2][i & 3]);
      __builtin_amdgcn_sched_barrier(0);
      if (i < 8) {
        f0[i] = frag(h + 1, 0, i);
      }
      if ((i & 3) == 3) {
        issue_one(hc, 4 + (i >> 2), h + 3);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<8>();  // this wave's copies of slice h + 2 have landed
    stage_barrier();  // everyone's have: slice h + 2 is readable, slot (h & 3) is free
  }
  wait_vmcnt<0>();    // no copy may still be writing LDS when the wave ends

#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
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
// 16-bit TN GEMM for grids of one to two 256x256 tiles per CU: the 4 waves of
// 128x128 of gemm_half_tn_w4_kernel over two 64-deep LDS stages with
// 128-byte rows (the swizzle of gemm_half_tn_lds_kernel), so each copy moves
// whole 128-byte lines.  Two barriers per stage: B1 at a stage's start
// (everyone is done with the other buffer, which the next stage's copies
// refill: 16 per wave, one after every second MFMA of k-steps 0 and 1) and
// B2 after k-step 2 (the wave has waited for its copies; the barrier makes
// the next stage readable), so k-step 3 already reads the next stage's first
// fragments.  Past the last stage the copies re-load it into the free buffer
// (unused).  Same k order per accumulator as the other two kernels
// (bit-identical results).  Measured on 4096^3 bf16: 1267-1289 TFLOP/s
// against 1240-1260 for gemm_half_tn_lds_kernel; on 8192^3 it trails
// gemm_half_tn_w4_kernel (1259-1284 against 1297-1310).
// ---------------------------------------------------------------------------
template <typename T, typename Epi>
__global__ __launch_bounds__(256) void gemm_half_tn_w4d_kernel(const uint16_t* __restrict__ A,
                                                               const uint16_t* __restrict__ Bt, int M, int N, int K,
                                                               int lda, int ldb, int tiles_n, Epi epi) {
  constexpr int BM = 256, BN = 256, BK = 64;
  constexpr int ROWB = BK * 2;            // bytes per LDS row (128)
  constexpr int STAGE = (BM + BN) * BK;   // elements per stage
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;

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
  const int bm = (first_m + in_group % gm) * BM;
  const int bn = (in_group / gm) * BN;

  // Copy instruction i (0..31 per operand per stage) fills rows 8i + lane/8,
  // physical chunk lane%8; wave w issues i = w + 4j, j = 0..7.
  const int crow = lane >> 3;
  const int pch = lane & 7;
  uint32_t a_off[8];
  uint32_t b_off[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = 8 * (wave + 4 * j) + crow;
    const int lch = pch ^ ((row >> 1) & 7);
    a_off[j] = static_cast<uint32_t>(row * lda + lch * 8) * 2u;
    b_off[j] = static_cast<uint32_t>(row * ldb + lch * 8) * 2u;
  }
  const uint16_t* a_tile = A + static_cast<size_t>(bm) * lda;
  const uint16_t* b_tile = Bt + static_cast<size_t>(bn) * ldb;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = lds_addr(smem);
  // Copy q (0..15) of stage kt into buffer buf: A rows for q < 8, then B.
  auto issue_one = [&](int kt, int q, int buf) {
    const uint32_t base = lds0 + 2u * static_cast<uint32_t>((buf & 1) * STAGE);
    const int k0 = kt * BK;
    if (q < 8) {
      load_lds16_sbase(a_off[q], a_tile + k0, base + static_cast<uint32_t>((wave_s + 4 * q) * 1024));
    } else {
      load_lds16_sbase(b_off[q - 8], b_tile + k0,
                       base + 2u * BM * BK + static_cast<uint32_t>((wave_s + 4 * (q - 8)) * 1024));
    }
  };

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  // Fragment f (0..7) of k-step s of the stage in buffer buf: A rows for
  // f < 4, then B rows.
  auto frag = [&](int buf, int s, int f) -> u32x4 {
    const char* base = reinterpret_cast<const char*>(smem + (buf & 1) * STAGE);
    const int row = f < 4 ? wm + f * 32 + lrow : wn + (f - 4) * 32 + lrow;
    const int opoff = f < 4 ? 0 : 2 * BM * BK;
    const int c = 2 * s + lhalf;
    return *reinterpret_cast<const u32x4*>(base + opoff + row * ROWB + ((c ^ ((row >> 1) & 7)) << 4));
  };

  floatx16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = zero16();
    }
  }

  const int nk = K / BK;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    issue_one(0, q, 0);
  }
  wait_vmcnt<0>();
  __builtin_amdgcn_s_waitcnt(0xc07f);  // no scalar load pending at the loop head
  stage_barrier();
  u32x4 f0[8];
  u32x4 f1[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    f0[f] = frag(0, 0, f);
  }
  for (int kt = 0; kt < nk; ++kt) {
    const int kc = min(kt + 1, nk - 1);
    stage_barrier();  // B1: everyone is done with buffer (kt + 1) & 1
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4(&cur)[8] = (s & 1) ? f1 : f0;
      u32x4(&nxt)[8] = (s & 1) ? f0 : f1;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        acc[i >> 2][i & 3] = mfma32x32x16<T>(cur[i >> 2], cur[4 + (i & 3)], acc[i >> 2][i & 3]);
        __builtin_amdgcn_sched_barrier(0);
        if (i < 8) {
          nxt[i] = s < 3 ? frag(kt, s + 1, i) : frag(kt + 1, 0, i);
        }
        if (s < 2 && (i & 1)) {
          issue_one(kc, s * 8 + (i >> 1), kt + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (s == 2) {
        wait_vmcnt<0>();  // this wave's copies of stage kt + 1 have landed
        stage_barrier();  // B2: everyone's have
      }
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
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
// 16-bit TN GEMM, 256x256 tile, 4 waves of 128x128 (one per SIMD), fed by a
// ring of 128-byte-row LDS parts.  A part is 128 rows x 64 k (16 KiB): stage
// s (k in [64s, 64s + 64)) is parts 4s..4s+3 = A rows 0-127, A rows 128-255,
// Bt rows 0-127, Bt rows 128-255, and part p lives in ring slot p % 10 (the
// ring is the whole 160 KiB of LDS).  Each global -> LDS copy moves 8 rows x
// 128 bytes, whole cache lines: the L1 sends one 128-byte request per row to
// L2 where the 64-byte rows of gemm_half_tn_w4_kernel's 32-deep slices sent
// two (counters on 8192^3: 136M L2 read requests against 67M for the same
// bytes, the address unit stalled on the L1 for 67M cycles).
//
// Per stage a wave runs 4 k-steps of 16 MFMAs (32x32x16).  Its 16 copies go
// to parts 4s+6 .. 4s+9 (the last two parts of stage s+1, the first two of
// stage s+2), whose slots held stage s-1: the first 8 one after every second
// MFMA of k-step 0, the rest one after every fourth MFMA of k-steps 1-2.
// Fragments of k-step j+1 are read during k-step j.  In k-step 3, after its
// first 8 MFMAs, the wave waits for its own copies of stage s+1 (vmcnt(8):
// only the 8 copies of stage s+2 may still be in flight) and meets the one
// barrier of the stage, which makes stage s+1 readable and retires stage s
// (whose last fragments are already in registers); it then issues the reads
// of stage s+1's first fragments, which land while the other 8 MFMAs run.  So a copy has at least 2.5
// k-steps to land, every stage has one barrier and no fragment read waits on
// one.  Copies past the last stage re-load it into retired slots (unused).
//
// The LDS rows carry the 128-byte swizzle of gemm_half_tn_lds_kernel (16-byte
// chunk c of row r at c ^ ((r >> 1) & 7)): the fragment reads of 16 rows
// touch every bank once.  The k order of each accumulator is that of the
// other 256x256 kernels (bit-identical results).  Tiles are ordered in groups
// of 4 tile rows per XCD.  Operands are padded to 256 rows; lane offsets are
// 32-bit (the host keeps 256 * ld * 2 bytes below 2^31).
// ---------------------------------------------------------------------------
template <typename T, typename Epi>
__global__ __launch_bounds__(256) void gemm_half_tn_w4r_kernel(const uint16_t* __restrict__ A,
                                                               const uint16_t* __restrict__ Bt, int M, int N, int K,
                                                               int lda, int ldb, int tiles_n, Epi epi) {
  constexpr int BM = 256, BN = 256, BK = 64;
  constexpr int ROWB = BK * 2;           // bytes per LDS row (128)
  constexpr int PART = 128 * BK;         // elements per part
  constexpr int NPART = 10;              // ring slots (160 KiB)
  __shared__ __attribute__((aligned(16))) uint16_t smem[NPART * PART];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;

  constexpr int GROUP = 4;
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
  const int bm = (first_m + in_group % gm) * BM;
  const int bn = (in_group / gm) * BN;

  // Copy instruction i (0..15 per part) fills part rows 8i + lane/8, physical
  // chunk lane%8; wave w issues i = w + 4j, j = 0..3.
  const int crow = lane >> 3;
  const int pch = lane & 7;
  uint32_t a_off[4];
  uint32_t b_off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * (wave + 4 * j) + crow;
    const int lch = pch ^ ((row >> 1) & 7);
    a_off[j] = static_cast<uint32_t>(row * lda + lch * 8) * 2u;
    b_off[j] = static_cast<uint32_t>(row * ldb + lch * 8) * 2u;
  }
  const uint16_t* a_tile = A + static_cast<size_t>(bm) * lda;
  const uint16_t* b_tile = Bt + static_cast<size_t>(bn) * ldb;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = lds_addr(smem);
  const int S = K / BK;
  // Copy j (0..3) of part p into slot `slot` (= p % NPART); parts past the
  // last stage re-load the last stage.
  auto issue_one = [&](int p, int slot, int j) {
    const int st = min(p >> 2, S - 1);
    const int ty = p & 3;
    const uint32_t dst = lds0 + static_cast<uint32_t>(slot * PART * 2 + (wave_s + 4 * j) * 1024);
    if (ty < 2) {
      load_lds16_sbase(a_off[j], a_tile + static_cast<size_t>(ty * 128) * lda + st * BK, dst);
    } else {
      load_lds16_sbase(b_off[j], b_tile + static_cast<size_t>((ty - 2) * 128) * ldb + st * BK, dst);
    }
  };

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  // Fragment f (0..7: A rows for f < 4, then Bt rows) of k-step kk of the
  // stage whose A / Bt parts of this wave sit in slots sa / sb.
  auto frag = [&](int sa, int sb, int kk, int f) -> u32x4 {
    const int slot = f < 4 ? sa : sb;
    const int row = (f & 3) * 32 + lrow;
    const int c = 2 * kk + lhalf;
    const char* base = reinterpret_cast<const char*>(smem + slot * PART);
    return *reinterpret_cast<const u32x4*>(base + row * ROWB + ((c ^ ((row >> 1) & 7)) << 4));
  };
  auto wrap = [](int x) { return x >= NPART ? x - NPART : x; };

  floatx16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = zero16();
    }
  }

  // Prologue: stage 0 and the first two parts of stage 1.
#pragma unroll
  for (int p = 0; p < 6; ++p) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      issue_one(p, p, j);
    }
  }
  wait_vmcnt<8>();                     // stage 0 has landed
  __builtin_amdgcn_s_waitcnt(0xc07f);  // no scalar load pending at the loop head
  stage_barrier();
  // slot of this stage's first part, and of this wave's A / Bt parts
  int s0 = 0;
  const int ta = wm >> 7;
  const int tb = 2 + (wn >> 7);
  u32x4 f0[8];
  u32x4 f1[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    f0[f] = frag(ta, tb, 0, f);
  }
  for (int s = 0; s < S; ++s) {
    const int sa = wrap(s0 + ta);
    const int sb = wrap(s0 + tb);
    const int p6 = 4 * s + 6;
    const int c6 = wrap(s0 + 6);  // slot of part 4s+6; parts 4s+6..4s+9 fill the slots of stage s-1
    // k-step 0: MFMAs on f0; f1 <- k-step 1; copies of parts 4s+6, 4s+7
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i >> 2][i & 3] = mfma32x32x16<T>(f0[i >> 2], f0[4 + (i & 3)], acc[i >> 2][i & 3]);
      __builtin_amdgcn_sched_barrier(0);
      if (i < 8) {
        f1[i] = frag(sa, sb, 1, i);
      }
      if (i & 1) {
        const int q = i >> 1;  // 0..7
        issue_one(p6 + (q >> 2), wrap(c6 + (q >> 2)), q & 3);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // k-step 1: MFMAs on f1; f0 <- k-step 2; copies of part 4s+8
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i >> 2][i & 3] = mfma32x32x16<T>(f1[i >> 2], f1[4 + (i & 3)], acc[i >> 2][i & 3]);
      __builtin_amdgcn_sched_barrier(0);
      if (i < 8) {
        f0[i] = frag(sa, sb, 2, i);
      }
      if ((i & 3) == 3) {
        issue_one(p6 + 2, wrap(c6 + 2), i >> 2);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // k-step 2: MFMAs on f0; f1 <- k-step 3; copies of part 4s+9
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i >> 2][i & 3] = mfma32x32x16<T>(f0[i >> 2], f0[4 + (i & 3)], acc[i >> 2][i & 3]);
      __builtin_amdgcn_sched_barrier(0);
      if (i < 8) {
        f1[i] = frag(sa, sb, 3, i);
      }
      if ((i & 3) == 3) {
        issue_one(p6 + 3, wrap(c6 + 3), i >> 2);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // k-step 3: 8 MFMAs, the stage barrier, then the next stage's first
    // fragments under the other 8 MFMAs.
    const int n0 = wrap(s0 + 4);
    const int na = wrap(n0 + ta);
    const int nb = wrap(n0 + tb);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[i >> 2][i & 3] = mfma32x32x16<T>(f1[i >> 2], f1[4 + (i & 3)], acc[i >> 2][i & 3]);
      __builtin_amdgcn_sched_barrier(0);
      if (i == 7) {
        wait_vmcnt<8>();  // this wave's copies of stage s + 1 have landed
        stage_barrier();  // everyone's have; stage s is retired
        // all 8 reads at once, A block 0 and the Bt blocks first (the next
        // stage's first four MFMAs use them), under the remaining 8 MFMAs
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int f = q == 0 ? 0 : (q <= 4 ? q + 3 : q - 4);
          f0[f] = frag(na, nb, 0, f);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    s0 = n0;
  }
  wait_vmcnt<0>();  // no copy may still be writing LDS when the wave ends

#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
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
// 16-bit TN GEMM, 256x256 tile, 4 waves of 128x128 (one per SIMD), with the
// fragments of a whole half stage held in registers (the default from 256
// tiles).  LDS is the ring of ten 16 KiB parts of gemm_half_tn_w4r_kernel
// (part p = stage p / 4, type p % 4: A rows 0-127, A rows 128-255, Bt rows
// 0-127, Bt rows 128-255; slot p % 10; 128-byte rows, chunk c of row r at
// c ^ ((r >> 1) & 7)), but each stage has its one barrier in the middle:
//   first half of stage s   MFMAs of k 0..31 from registers r0, while the
//                           fragments of k 32..63 of stage s are read into r1;
//   barrier                 this wave's copies of stage s + 1 have landed and
//                           its reads of stage s are done (so stage s retires);
//   second half             MFMAs of k 32..63 from r1, while k 0..31 of stage
//                           s + 1 are read into r0.
// A fragment read thus has half a stage (64 MFMAs) to land, and no MFMA waits
// on a barrier.  The copies of stage s + 2 go out one per 8 MFMAs over the
// whole stage: its A parts during the first half into the slots stage s - 1
// left, its Bt parts after the barrier into stage s's, so every copy has at
// least a half stage before the barrier that waits for it.
//
// v_mfma_f32_16x16x32 (8 x 8 blocks of 16x16 per wave, 64 MFMAs per 32-deep
// k-step): measured against the same schedule on 32x32x16 at 8192^3, 1463 vs
// 1386 TFLOP/s on one box; the per-element k order is unchanged (results are
// bit-identical to the other 256x256 kernels).  The Bt fragment is the MFMAs'
// A operand, so each lane accumulates 4 consecutive columns of one C row and
// the epilogue stores 16 bytes per block (4096^3: 97.5 -> 96.0 us; 8192^3
// unchanged).  Copy j (0..3) of wave w for
// one part fills part rows 32w + 8j .. + 7: the four copies share one M0 and
// one SALU copy of the base pair, and step by the instruction offset.  The
// stage bodies are unrolled by five (the
// ring's period), so every slot is a constant and every fragment read is one
// ds_read_b128 with an immediate offset from one of six lane bases.
// Operands padded to 256 rows and K to 64; lane offsets are 32-bit (the host
// keeps 256 * ld * 2 bytes below 2^31).
// ---------------------------------------------------------------------------
template <typename T, typename Epi>
__global__ __launch_bounds__(256) void gemm_half_tn_w4h_kernel(const uint16_t* __restrict__ A,
                                                               const uint16_t* __restrict__ Bt, int M, int N, int K,
                                                               int lda, int ldb, int tiles_n, Epi epi) {
  constexpr int BM = 256, BN = 256, BK = 64;
  constexpr int PARTB = 128 * BK * 2;  // bytes per part
  constexpr int NPART = 10;
  __shared__ __attribute__((aligned(16))) uint16_t smem[NPART * PARTB / 2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;

  constexpr int GROUP = 4;
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
  const int bm = (first_m + in_group % gm) * BM;
  const int bn = (in_group / gm) * BN;

  // Copy offsets [half][j] (the instruction offset 1024 * j moves both
  // addresses, so it is taken off the global one; rows >= 8j keep them >= 0).
  const int crow = lane >> 3;
  const int pch = lane & 7;
  uint32_t a_off[2][4];
  uint32_t b_off[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 32 * wave + 8 * j + crow;
    const int lch = pch ^ ((row >> 1) & 7);
    a_off[0][j] = static_cast<uint32_t>(row * lda + lch * 8) * 2u - 1024u * j;
    b_off[0][j] = static_cast<uint32_t>(row * ldb + lch * 8) * 2u - 1024u * j;
    a_off[1][j] = a_off[0][j] + static_cast<uint32_t>(128 * lda) * 2u;
    b_off[1][j] = b_off[0][j] + static_cast<uint32_t>(128 * ldb) * 2u;
  }
  const char* a_tile = reinterpret_cast<const char*>(A + static_cast<size_t>(bm) * lda);
  const char* b_tile = reinterpret_cast<const char*>(Bt + static_cast<size_t>(bn) * ldb);
  const uint32_t wave_lds = lds_addr(smem) + static_cast<uint32_t>(wave) * 4096u;
  const int S = K / BK;
  // Copy j of part p (its stage clamped to the last: past the end a retired
  // slot is refilled with the last stage, unused) into `slot`.  Copy 0 of a
  // part makes the SALU copy of its base pair in `pair`; copies 1-3 read it.
  auto copy_pj = [&](uint64_t& pair, int p, int slot, int j) {
    const int ty = p & 3;
    const uint32_t voff = ty < 2 ? a_off[ty][j] : b_off[ty - 2][j];
    const uint32_t m0 = wave_lds + static_cast<uint32_t>(slot * PARTB);
    switch (j) {
      case 0: {
        const int st = min(p >> 2, S - 1);
        pair = load_lds16_sbase_first(voff, (ty < 2 ? a_tile : b_tile) + st * (BK * 2), m0);
        break;
      }
      case 1: load_lds16_pair_off<1024>(voff, pair, m0); break;
      case 2: load_lds16_pair_off<2048>(voff, pair, m0); break;
      default: load_lds16_pair_off<3072>(voff, pair, m0); break;
    }
  };

  // Fragment reads: lane l reads row l % 16 of a 16-row block, 16-byte chunk
  // 4 * kk + l / 16 of k-step kk (0, 1) of the stage.  Bases rb[kk][q] =
  // that lane part + q * 64 KiB; slot and block go into the immediate.
  const int lrow = lane & 15;
  const int lq = lane >> 4;
  typedef __attribute__((address_space(3))) const char lds_char;
  typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
  lds_char* lbase = (lds_char*)(smem);
  lds_char* rb[2][3];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    lds_char* o = lbase + (lrow * 128 + (((4 * kk + lq) ^ ((lrow >> 1) & 7)) << 4));
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      rb[kk][q] = o + q * 65536;
    }
  }
  const int ta = wm >> 7;        // this wave's A part type
  const int tb = 2 + (wn >> 7);  // and Bt part type
  // fragment f (0..7: A row blocks of 16, 8..15: Bt) of k-step kk of `slot`
  auto frag = [&](int slot, int kk, int f) -> u32x4 {
    const int byte = slot * PARTB + (f & 7) * 2048;
    return *reinterpret_cast<lds_u32x4*>(rb[kk][byte >> 16] + (byte & 0xffff));
  };

  floatx4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }

  // Prologue: stages 0 and 1 (parts 0-7 into slots 0-7), then the first k-step
  // of stage 0 into registers.
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    uint64_t pair;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      copy_pj(pair, p, p, j);
    }
  }
  wait_vmcnt<16>();                    // stage 0 has landed
  __builtin_amdgcn_s_waitcnt(0xc07f);  // no scalar load pending at the loop head
  stage_barrier();
  u32x4 r0[16];
  u32x4 r1[16];
#pragma unroll
  for (int f = 0; f < 16; ++f) {
    r0[f] = frag(f < 8 ? ta : tb, 0, f);
  }

  auto body = [&](auto phase, int s) {
    constexpr int t = decltype(phase)::value;  // s % 5
    constexpr int sl0 = (4 * t) % NPART;       // slot of part 4s
    constexpr int nsl = (4 * t + 4) % NPART;   // slot of part 4s + 4
    uint64_t pair = 0;                         // base pair of the part being copied
    // first half: k-step 0 on r0; r1 <- k-step 1; copies of parts 4s+8, 4s+9
#pragma unroll
    for (int g = 0; g < 64; ++g) {
      acc[g >> 3][g & 7] = mfma16x16x32<T>(r0[8 + (g & 7)], r0[g >> 3], acc[g >> 3][g & 7]);
      __builtin_amdgcn_sched_barrier(0);
      if ((g & 1) == 0 && g < 32) {
        const int f = g >> 1;
        r1[f] = frag((sl0 + (f < 8 ? ta : tb)) % NPART, 1, f);
      }
      if ((g & 7) == 4) {
        const int c = g >> 3;
        copy_pj(pair, 4 * s + 8 + (c >> 2), (sl0 + 8 + (c >> 2)) % NPART, c & 3);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<8>();    // this wave's copies of stage s + 1 have landed
    wait_lgkmcnt<0>();  // and its reads of stage s are done
    stage_barrier();    // everyone's: stage s + 1 is readable, stage s retires
    // second half: k-step 1 on r1; r0 <- k-step 0 of stage s+1; copies of
    // parts 4s+10, 4s+11
#pragma unroll
    for (int g = 0; g < 64; ++g) {
      acc[g >> 3][g & 7] = mfma16x16x32<T>(r1[8 + (g & 7)], r1[g >> 3], acc[g >> 3][g & 7]);
      __builtin_amdgcn_sched_barrier(0);
      if ((g & 3) == 0) {
        const int f = g >> 2;
        r0[f] = frag((nsl + (f < 8 ? ta : tb)) % NPART, 0, f);
      }
      if ((g & 7) == 4) {
        const int c = g >> 3;
        copy_pj(pair, 4 * s + 10 + (c >> 2), (sl0 + 10 + (c >> 2)) % NPART, c & 3);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int s = 0; s < S; s += 5) {
    body(std::integral_constant<int, 0>{}, s);
    if (s + 1 < S) body(std::integral_constant<int, 1>{}, s + 1);
    if (s + 2 < S) body(std::integral_constant<int, 2>{}, s + 2);
    if (s + 3 < S) body(std::integral_constant<int, 3>{}, s + 3);
    if (s + 4 < S) body(std::integral_constant<int, 4>{}, s + 4);
  }
  wait_vmcnt<0>();  // no copy may still be writing LDS

  // acc[i][j] holds rows i*16 + lane % 16 and columns j*16 + 4*(lane / 16) ..
  // + 3 of the wave's C block (the MFMAs take the Bt fragment as their A
  // operand, so they accumulate C^T).  Stored straight from there, one store
  // instruction covers 16 rows x 64 bytes; instead each wave stages its
  // 128 x 128 block through its own 40 KB of the (now idle) ring in two
  // 64-row chunks (rows of 132 floats: the 16 rows of a ds_write_b128 hit
  // distinct banks) and reads it back 2 rows x 512 bytes per instruction, so
  // every store writes 8 whole 128-byte lines.  Measured at 8192^3 (bits
  // unchanged): 1576 against 1541 TFLOP/s; 4096^3 unchanged (its one round
  // of stores is bound by HBM writes).
  __builtin_amdgcn_s_waitcnt(0xc07f);
  stage_barrier();  // every wave is done reading the ring
  typedef __attribute__((address_space(3))) float lds_float;
  typedef __attribute__((address_space(3))) floatx4 lds_floatx4;
  lds_float* stg = (lds_float*)(smem) + wave * 10240;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        *reinterpret_cast<lds_floatx4*>(stg + (16 * i + lrow) * 132 + 16 * j + 4 * lq) = acc[4 * c + i][j];
      }
    }
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      const int r = 2 * t + (lane >> 5);
      const int col = 4 * (lane & 31);
      const floatx4 val = *reinterpret_cast<lds_floatx4*>(stg + r * 132 + col);
      const int m = bm + wm + 64 * c + r;
      if (m < M) {
        epi.store4(m, bn + wn + col, N, val);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Ring-pipelined 16-bit TN GEMM for short K (the ViT block's GEMMs, K = 768).
//
// With K = 768 a tile has 12 stages of BK = 64 and each stage holds only a
// few MFMAs per wave, so a loop that prefetches one stage ahead pays a global
// load latency per stage.  Here NS stages of LDS form a ring and the copies of
// stage s + NS - 1 go out when stage s starts: one latency per tile.
// Copies are scalar-base global -> LDS (load_lds16_sbase) with the 128-byte
// row swizzle of gemm_half_tn_lds_kernel; per-lane offsets are fixed for the
// tile and rows past M (or N) are clamped to the last row (read, computed,
// never stored).  The A source is a policy: row-major, or the implicit
// im2col of a patch-embedding convolution.
// ---------------------------------------------------------------------------

// Row-major A [M, lda]: stage base = tile row bm, column k0.
struct RingRowMajor {
  const uint16_t* A;
  int lda;
  __device__ __forceinline__ const uint16_t* stage_base(int bm, int k0) const {
    return A + static_cast<size_t>(bm) * lda + k0;
  }
  // Byte offset of (row, k0 + kk) from stage_base(bm, k0), row in [bm, M).
  __device__ __forceinline__ uint32_t lane_offset(int bm, int row, int kk) const {
    return static_cast<uint32_t>((row - bm) * lda + kk) * 2u;
  }
};

// Implicit im2col of a patch-embedding convolution (kernel = stride = P, no
// padding) over x [B, C, H, W]: row = b*T + ty*gw + tx, k = (c*P + ky)*P + kx.
// With P dividing BK and BK dividing P*P a BK-wide stage is BK/P kernel rows
// of one channel: k0 fixes (c, first ky) for every lane (the stage base) and
// the lane adds its patch origin plus kk / P rows and kk % P columns.
struct RingPatch {
  const uint16_t* x;
  int C, H, W, P, T, gw;
  __device__ __forceinline__ const uint16_t* stage_base(int, int k0) const {
    const int pp = P * P;
    const int c = k0 / pp;
    const int ky0 = (k0 - c * pp) / P;
    return x + (static_cast<size_t>(c) * H + ky0) * W;
  }
  __device__ __forceinline__ uint32_t lane_offset(int, int row, int kk) const {
    const int b = row / T;
    const int t = row - b * T;
    const int ty = t / gw;
    const int tx = t - ty * gw;
    const int origin = ((b * C) * H + ty * P) * W + tx * P;
    return static_cast<uint32_t>(origin + (kk / P) * W + kk % P) * 2u;
  }
};

// BK = 64 (128-byte LDS rows, chunk c of row r at c ^ ((r >> 1) & 7)) or
// BK = 128 (256-byte rows, chunk c at c ^ (r & 15)): each 1 KB copy then
// fills 8 or 4 rows.  The deeper stage halves the per-stage waits and
// barriers: in the ViT block (K = 768, 128x64 tiles, three 48 KiB stages)
// the patch GEMM went 9.5 -> 8.8 us and the output projection 7.8 -> 7.3 us
// (kernel trace); the k order, and so the result, is unchanged.
template <typename T, int BM, int BN, int WM, int WN, int NS, typename ASrc, typename Epi, int BK = 64>
__global__ __launch_bounds__(WM* WN * 64) void gemm_half_ring_kernel(ASrc asrc, const uint16_t* __restrict__ Bt,
                                                                       int M, int N, int K, int ldb, int tiles_n,
                                                                       Epi epi) {
  static_assert(BK == 64 || BK == 128, "stage depth");
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM / 32;
  constexpr int TN = BN / WN / 32;
  constexpr int ROWB = BK * 2;                 // bytes per LDS row
  constexpr int RPI = 1024 / ROWB;             // rows per 1 KB copy
  constexpr int CPR = ROWB / 16;               // 16-byte chunks per row
  constexpr int STAGE = (BM + BN) * BK;        // elements per stage
  constexpr int A_INS = BM / RPI;              // 1 KB copies of A per stage
  constexpr int LPW = (BM + BN) / RPI / NW;    // copies per wave per stage
  constexpr int A_LPW = A_INS / NW;            // ... of which A
  static_assert(TM >= 1 && TN >= 1 && A_INS % NW == 0 && (BN / RPI) % NW == 0, "tile / wave split");
  static_assert(NS >= 2 && NS <= 5 && NS * STAGE * 2 <= 160 * 1024, "LDS ring");
  static_assert(3 * LPW < 64, "vmcnt immediate");
  __shared__ __attribute__((aligned(16))) uint16_t smem[NS * STAGE];
  auto swz = [](int r) { return BK == 64 ? ((r >> 1) & 7) : (r & 15); };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave / WN) * (BM / WM);
  const int wn = (wave % WN) * (BN / WN);

  // XCD-aware tile order.  Workgroup w runs on XCD w % 8, so the remap gives
  // XCD x the contiguous range [x * n / 8, (x + 1) * n / 8) of the order
  // below: the tile columns split into two halves and, within a half, tiles
  // go row by row.  XCDs 0-3 then cover the first half's columns and XCDs
  // 4-7 the second's, each about a quarter of the tile rows: an XCD's L2
  // misses a quarter of A and half of B (one round of 156 workgroups in the
  // ViT block's N = 768 GEMMs: 11.4 MB read past L2 per GEMM, where groups
  // of 8 tile rows over every column read A about eight times, 14.7 MB).
  const int tiles_m = (M + BM - 1) / BM;
  const int full = static_cast<int>(gridDim.x) & ~7;
  int pid = blockIdx.x;
  if (pid < full) {
    pid = (pid & 7) * (full >> 3) + (pid >> 3);
  }
  const int half_n = (tiles_n + 1) / 2;
  const int first_half = tiles_m * half_n;
  int bm, bn;
  if (pid < first_half) {
    bm = (pid / half_n) * BM;
    bn = (pid % half_n) * BN;
  } else {
    const int rest = tiles_n - half_n;
    const int q = pid - first_half;
    bm = (q / rest) * BM;
    bn = (half_n + q % rest) * BN;
  }

  // Copy j of this wave is instruction i = wave + NW*j: A rows RPI*i ..
  // RPI*i + RPI-1 for j < A_LPW, else B rows RPI*(i - A_INS)..; lane l ->
  // row + l/CPR, physical chunk l%CPR, logical chunk (l%CPR) ^ swz(row).
  uint32_t off[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int ins = wave + NW * j;
    const int r = RPI * (j < A_LPW ? ins : ins - A_INS) + lane / CPR;
    const int kk = ((lane % CPR) ^ swz(r)) * 8;
    if (j < A_LPW) {
      off[j] = asrc.lane_offset(bm, min(bm + r, M - 1), kk);
    } else {
      off[j] = static_cast<uint32_t>((min(bn + r, N - 1) - bn) * ldb + kk) * 2u;
    }
  }
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = lds_addr(smem);
  const uint16_t* b_tile = Bt + static_cast<size_t>(bn) * ldb;
  auto issue = [&](int buf, int k0) {
    const uint16_t* a_base = asrc.stage_base(bm, k0);
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const uint32_t dst = lds0 + 2u * static_cast<uint32_t>(buf * STAGE + (wave_s + NW * j) * RPI * BK);
      load_lds16_sbase(off[j], j < A_LPW ? a_base : b_tile + k0, dst);
    }
  };

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  auto frag = [&](const uint16_t* base, int row, int c) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + row * ROWB + ((c ^ swz(row)) << 4));
  };
  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      acc[i][j] = zero16();
    }
  }

  const int nk = K / BK;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) {
    if (s < nk) {
      issue(s, s * BK);
    }
  }
  // Only LDS reads may be outstanding in the loop (a pending scalar load
  // would make every fragment wait an lgkmcnt(0)).
  __builtin_amdgcn_s_waitcnt(0xc07f);
  int buf = 0;
  for (int kt = 0; kt < nk; ++kt) {
    // Stage kt has landed (this wave's copies) once at most the later
    // stages' copies are outstanding; the barrier extends that to every wave
    // and retires everyone's reads of stage kt-1, whose buffer is refilled.
    const int later = min(NS - 2, nk - 1 - kt);
    if (later >= 3) {
      wait_vmcnt<3 * LPW>();
    } else if (later == 2) {
      wait_vmcnt<2 * LPW>();
    } else if (later == 1) {
      wait_vmcnt<LPW>();
    } else {
      wait_vmcnt<0>();
    }
    stage_barrier();
    if (kt + NS - 1 < nk) {
      issue(buf == 0 ? NS - 1 : buf - 1, (kt + NS - 1) * BK);
    }
    const uint16_t* As = smem + buf * STAGE;
    const uint16_t* Bs = As + BM * BK;
    u32x4 af[2][TM];
    u32x4 bf[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      af[0][i] = frag(As, wm + i * 32 + lrow, lhalf);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      bf[0][j] = frag(Bs, wn + j * 32 + lrow, lhalf);
    }
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int cur = s & 1;
      if (s + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          af[cur ^ 1][i] = frag(As, wm + i * 32 + lrow, 2 * (s + 1) + lhalf);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          bf[cur ^ 1][j] = frag(Bs, wn + j * 32 + lrow, 2 * (s + 1) + lhalf);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          acc[i][j] = mfma32x32x16<T>(af[cur][i], bf[cur][j], acc[i][j]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    buf = buf + 1 == NS ? 0 : buf + 1;
  }

#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = bn + wn + j * 32 + lrow;
      if constexpr (AccStore<Epi>::value) {
        epi.store_acc(bm + wm + i * 32, n, acc[i][j], lane, M, N);
      } else {
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
}

// ---------------------------------------------------------------------------
// fp32 GEMM on padded operands: direct global -> LDS loads, stream-K.
//
// 64x64 block tile, 4*KS waves: each group of 4 waves covers the four 32x32
// output sub-tiles on its 1/KS of every K stage (KS waves per SIMD, so one
// wave's LDS waits hide behind the others' MFMAs); the KS parts are summed
// through LDS at the end of a tile.  BK = 32 or 64 per
// stage, STAGES buffers, loads issued STAGES-1 stages ahead, one wait +
// barrier per stage.
//
// LDS: A stage [64 m][BK k] with the 16-byte chunks of each row XOR-swizzled
// (by row & 15 for 256-byte rows, (row >> 1) & 7 for 128-byte rows), so the
// 16 rows one 16-byte read serves per clock (256 bytes, 64 banks) hit 16
// different bank groups; B stage [BK k][64 n] with the two 128-byte halves of
// every row that has bit 2 set swapped.  v_mfma_f32_32x32x2_f32 takes one k
// pair per lane half; with the k permutation "MFMA j of an 8-k group uses
// k = 8c + j (lanes 0-31) and 8c + 4 + j (lanes 32-63)", a lane's four A
// values of a group are one 16-byte LDS read, and its B values are four
// 4-byte reads in which the two half-waves (rows 4 apart) use opposite bank
// halves.
//
// Work split (stream-K): the T*nk (tile, k-stage) iterations are divided
// evenly over the G workgroups, workgroup w taking [w*I/G, (w+1)*I/G).  A
// workgroup walks its range downwards, so the first segment it finishes is
// the low-k part of its last tile and the last segment the high-k part of
// its first tile.  A segment without the tile's last k stage publishes its
// partial tile (part[w], flag[w] = epoch) as soon as it is done; the segment
// holding the last stage owns the tile: it waits for the flags of the lower
// workgroups that hold the rest, adds their partials in workgroup order
// (deterministic) and stores.  With xl set, each XCD's workgroups split only
// the iterations of that XCD's own contiguous range of tiles (the same
// protocol among the ranks of one XCD).  Waits only ever target lower workgroup ids,
// which the in-order dispatch has already started, and each wait polls at
// most spin_limit times, so every wave exits.  An owner whose wait runs out
// stores 1 to *fail (the host turns it into an error after the stream sync)
// and stops waiting: that launch's result is invalid.  Flags carry the
// launch's epoch, a number the host changes on every launch, so a flag left
// by an earlier launch (one whose owner gave up before a late publisher set
// it) never reads as ready.  Owners clear the flags they saw set, so a launch
// without a timeout leaves every flag at zero and a replay of a captured
// launch (same epoch) starts clean.  With T a multiple of G (1024^3: 256
// tiles on 256 CUs) every range is whole tiles and nothing is published.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
  stage_barrier();
}

template <int BK, int STAGES, int KS, bool SK, typename Epi>
__global__ __launch_bounds__(256 * KS) void gemm_f32_lds_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                           int M, int N, int lda, int ldb, int tiles_m, int tiles_n,
                                                           int nk, StreamKSync sync, Epi epi, int xl = 0) {
  constexpr int BM = 64, BN = 64;
  constexpr int A_STAGE = BM * BK;            // floats
  constexpr int STAGE = (BM + BN) * BK;       // floats
  constexpr int ACH = BK / 4;                 // 16-byte chunks per A row
  constexpr int A_RPI = 64 / ACH;             // A rows per 1 KB load instruction
  constexpr int NW = 4 * KS;                  // waves
  constexpr int LPW = BK / 4 / NW;            // load instructions per wave per operand per stage
  constexpr int GPW = BK / 8 / KS;            // 8-k groups per wave per stage
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(LPW >= 1 && (BK / 4) % NW == 0 && GPW >= 1, "K split");
  __shared__ __attribute__((aligned(16))) float smem[STAGES * STAGE + (KS - 1) * 4096];
  auto swz = [](int row) { return ACH == 16 ? (row & 15) : ((row >> 1) & 7); };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = wave & 3;
  const int kh = wave >> 2;
  const int wm = (sub >> 1) * 32;
  const int wn = (sub & 1) * 32;

  const int G = gridDim.x;
  const int w = blockIdx.x;
  const int T = tiles_m * tiles_n;
  // XCD-local stream-K (xl, G % 8 == 0, T >= 8): workgroup w runs on XCD
  // w % 8; the G / 8 workgroups of an XCD (rank w / 8) split the iterations
  // of that XCD's own contiguous range of tiles, so operand tiles, partials
  // and flags stay in one L2.  Otherwise one range over all tiles.
  const int xcd = xl ? (w & 7) : 0;
  const int rank = xl ? (w >> 3) : w;
  const int Gs = xl ? (G >> 3) : G;
  const int tile0 = xl ? xcd * T / 8 : 0;
  const int Ts = xl ? (xcd + 1) * T / 8 - tile0 : T;
  const long long I = static_cast<long long>(Ts) * nk;
  auto begin_of = [&](int q) { return static_cast<int>(static_cast<long long>(q) * I / Gs); };
  auto wg_of = [&](int q) { return xl ? q * 8 + xcd : q; };
  // !SK: one whole tile per workgroup (G == T), no partials.
  const int it0 = SK ? begin_of(rank) : w * nk;
  const int it1 = SK ? begin_of(rank + 1) : it0 + nk;
  const int n_it = it1 - it0;
  if (n_it <= 0) {
    return;
  }

  // Tile t -> (bm, bn).  XCD-aware: consecutive tile ids (consecutive
  // workgroups) land on different XCDs, so pid = (t % 8) * (T / 8) + t / 8
  // gives each XCD a contiguous pid range, walked in groups of 8 tile rows.
  auto origin = [&](int t, int& bm, int& bn) {
    const int full = T & ~7;
    int pid = tile0 + t;
    if (!xl && pid < full) {
      pid = (pid & 7) * (full >> 3) + (pid >> 3);
    }
    const int group_size = 8 * tiles_n;
    const int group = pid / group_size;
    const int first_m = group * 8;
    const int gm = min(tiles_m - first_m, 8);
    const int in_group = pid - group * group_size;
    bm = (first_m + in_group % gm) * BM;
    bn = (in_group / gm) * BN;
  };

  // Wave w issues A instructions w + NW*j (A_RPI rows each) and B
  // instructions w + NW*j (4 k-rows of 256 bytes each), j < LPW; byte
  // offsets within a tile, fixed for all stages (the host keeps
  // 64 * ld * 4 bytes below 2^31).
  uint32_t a_off[LPW];
  uint32_t b_off[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int ins = wave + NW * j;
    const int row = A_RPI * ins + lane / ACH;
    const int lch = (lane % ACH) ^ swz(row);
    a_off[j] = static_cast<uint32_t>(row * lda + lch * 4) * 4u;
    const int krow = 4 * ins + (lane >> 4);
    b_off[j] = static_cast<uint32_t>(krow * ldb + ((lane & 15) ^ (krow & 4 ? 8 : 0)) * 4) * 4u;
  }
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = lds_addr(smem);
  // Issue cursor: next (tile, k) to load, walking down from it1 - 1.
  int is_t = (it1 - 1) / nk;
  int is_k = (it1 - 1) - is_t * nk;
  int is_bm, is_bn;
  origin(is_t, is_bm, is_bn);
  // Copy q of the cursor's stage into buffer buf: A for q < LPW, then B.
  auto issue_copy = [&](int buf, int q) {
    const uint32_t base = lds0 + 4u * static_cast<uint32_t>(buf * STAGE);
    if (q < LPW) {
      const float* a_base = A + static_cast<size_t>(is_bm) * lda + is_k * BK;
      load_lds16_sbase(a_off[q], a_base, base + 4u * static_cast<uint32_t>((wave_s + NW * q) * 256));
    } else {
      const float* b_base = B + static_cast<size_t>(is_k) * BK * ldb + is_bn;
      load_lds16_sbase(b_off[q - LPW], b_base,
                       base + 4u * static_cast<uint32_t>(A_STAGE + (wave_s + NW * (q - LPW)) * 256));
    }
  };
  auto advance = [&]() {
    if (--is_k < 0) {
      is_k = nk - 1;
      if (--is_t >= 0) {
        origin(is_t, is_bm, is_bn);
      }
    }
  };
  auto issue_next = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 2 * LPW; ++q) {
      issue_copy(buf, q);
    }
    advance();
  };

  floatx16 acc0 = zero16();
  floatx16 acc1 = zero16();
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) {
    if (s < n_it) {
      issue_next(s);
    }
  }
  const int arow = wm + (lane & 31);
  const int half = lane >> 5;
  float* red = smem + STAGES * STAGE + sub * 1024 + lane;

  // Segment end: sum the K parts, then publish, or own and store.
  auto finish = [&](int t, bool has_first, bool has_last) {
    if (kh > 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        red[(kh - 1) * 4096 + i * 64] = acc0[i] + acc1[i];
      }
    }
    lds_barrier();
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      v[i] = acc0[i] + acc1[i];
#pragma unroll
      for (int q = 0; q < KS - 1; ++q) {
        v[i] += red[q * 4096 + i * 64];
      }
    }
    // Partials and flags move with device-scope (sc1) loads and stores,
    // which are coherent across the XCDs' L2s by themselves; a release /
    // acquire fence instead would write back and invalidate the whole L2 of
    // the XCD and cost every other workgroup there its cached A / B tiles.
    // Order comes from waiting for the partial stores to complete (vmcnt)
    // before the flag store, and from the barrier after the flag spin.
    float* mine = sync.part + static_cast<size_t>(w) * 4096 + sub * 1024 + lane;
    if (!has_last) {
      if (kh == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          __hip_atomic_store(mine + i * 64, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      wait_vmcnt<0>();
      stage_barrier();
      if (tid == 0) {
        __hip_atomic_store(sync.flags + w, sync.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return;
    }
    if (!has_first) {
      int wf = static_cast<int>(static_cast<long long>(t) * nk * Gs / I);
      while (wf + 1 < Gs && begin_of(wf + 1) <= t * nk) {
        ++wf;
      }
      while (wf > 0 && begin_of(wf) > t * nk) {
        --wf;
      }
      int q_ready = rank;  // (wave 0, lane 0) flags [wf, q_ready) were seen set
      if (tid == 0) {
        for (int q = wf; q < rank; ++q) {
          if (begin_of(q) == begin_of(q + 1)) {
            continue;
          }
          const int* flag = sync.flags + wg_of(q);
          int spin = 0;
          while (spin < sync.spin_limit &&
                 __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != sync.epoch) {
            __builtin_amdgcn_s_sleep(4);
            ++spin;
          }
          if (spin >= sync.spin_limit) {
            // gave up: report, and wait for no further partial
            __hip_atomic_store(sync.fail, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            q_ready = q;
            break;
          }
        }
        // Clear the flags seen set, so a launch leaves its flags at zero
        // (a graph replay reuses the captured epoch).  A flag a late
        // publisher sets after a timeout keeps this launch's epoch, which no
        // later launch on these flags waits for.
        for (int q = wf; q < q_ready; ++q) {
          __hip_atomic_store(sync.flags + wg_of(q), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      stage_barrier();
      if (kh == 0) {
        for (int q = wf; q < rank; ++q) {
          float* theirs = sync.part + static_cast<size_t>(wg_of(q)) * 4096 + sub * 1024 + lane;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            v[i] += __hip_atomic_load(theirs + i * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
    }
    if (kh == 0) {
      int bm, bn;
      origin(t, bm, bn);
      const int n = bn + wn + (lane & 31);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = bm + wm + acc_row(i, lane);
        if (m < M && n < N) {
          epi(m, n, v[i]);
        }
      }
    }
  };

  int ct = (it1 - 1) / nk;
  int ck = (it1 - 1) - ct * nk;
  bool seg_has_last = ck == nk - 1;
  // Only LDS reads may be outstanding in the loop: a pending scalar load
  // would make every fragment wait an lgkmcnt(0).
  __builtin_amdgcn_s_waitcnt(0xc07f);
  for (int j = 0; j < n_it; ++j) {
    // Stage j's loads (own) have landed once at most min(n_it-1-j, STAGES-2)
    // later stages are outstanding; the barrier extends that to every wave
    // and retires the reads of stage j-1, whose buffer is refilled next.
    const int later = min(n_it - 1 - j, STAGES - 2);
    if (later >= 2) {
      wait_vmcnt<4 * LPW>();
    } else if (later == 1) {
      wait_vmcnt<2 * LPW>();
    } else {
      wait_vmcnt<0>();
    }
    stage_barrier();
    // The next stage's copies go out one after every second MFMA of this
    // stage's first half (a burst behind the barrier queues every wave's
    // copies at once); the cursor advances after the last one.
    const bool more = j + STAGES - 1 < n_it;
    const int nbuf = (j + STAGES - 1) % STAGES;
    const float* As = smem + (j % STAGES) * STAGE;
    const float* Bs = As + A_STAGE;
    floatx4 a[GPW];
    float b[GPW][4];
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
      const int c = kh * GPW + g;
      const int lch = 2 * c + half;
      a[g] = *reinterpret_cast<const floatx4*>(As + arow * BK + ((lch ^ swz(arow)) << 2));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        b[g][q] = Bs[(8 * c + 4 * half + q) * BN + ((wn + (lane & 31)) ^ (half << 5))];
      }
    }
    // All of the stage's fragment reads go out before its first MFMA (the
    // scheduler would otherwise pair each group's reads with its MFMAs and
    // expose the LDS latency once per group).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (u % 2 == 0) {
          acc0 = mfma32x32x2f32(a[g][u], b[g][u], acc0);
        } else {
          acc1 = mfma32x32x2f32(a[g][u], b[g][u], acc1);
        }
        const int mi = 4 * g + u;
        if (mi % 2 == 1 && mi / 2 < 2 * LPW && more) {
          __builtin_amdgcn_sched_barrier(0);
          issue_copy(nbuf, mi / 2);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    if (more) {
      advance();
    }
    if constexpr (SK) {
      if (ck == 0 || j == n_it - 1) {
        finish(ct, ck == 0, seg_has_last);
        acc0 = zero16();
        acc1 = zero16();
        seg_has_last = true;
      }
      if (--ck < 0) {
        ck = nk - 1;
        --ct;
      }
    }
  }
  if constexpr (!SK) {
    finish(w, true, true);
  }
}

// Tile configurations (block tile BM x BN, waves WM x WN, BK = 64):
//   w4     256x256, 4 waves 2x2 (128x128 each), ring of 32-deep slices
//          (gemm_half_tn_w4_kernel); needs A / Bt padded to 256 rows
//   w4d    256x256, 4 waves 2x2, two 64-deep stages, two barriers per stage
//          (gemm_half_tn_w4d_kernel); needs A / Bt padded to 256 rows
//   w4h    256x256, 4 waves 2x2, w4r's ring with the barrier mid-stage and a
//          half stage of fragments in registers, 16x16x32 MFMAs
//          (gemm_half_tn_w4h_kernel); needs A / Bt padded
//   w4r    256x256, 4 waves 2x2, ring of ten 128-byte-row parts, one barrier
//          per 64-deep stage (gemm_half_tn_w4r_kernel); needs A / Bt padded
//   lds    256x256, 8 waves 2x4 (128x64 each), global -> LDS direct loads
//          (gemm_half_tn_lds_kernel); needs A / Bt padded to 256 rows
//   big8   256x256, 8 waves 2x4, LDS double buffer fed from registers
//   big4   256x256, 4 waves 2x2 (128x128 each), 1 wave / SIMD
//   mid    128x128, 4 waves 2x2 (64x64 each)
//   small   64x64,  4 waves 2x2 (32x32 each)
// Default: the largest tile that still gives at least one workgroup per CU
// (w4h from one tile per CU where the operands are padded, big8 elsewhere).
// Alternating runs on one box, 8192^3 / 4096^3 bf16 TFLOP/s: w4h 1516-1529 /
// 1464-1467, w4r 1387-1390 / 1302-1307 (w4h since: 16-byte C stores and one
// base copy per part, 1555 / 1514 against w4r 1393 / 1319 on another box).
// Earlier, with alternating runs on one box, 8192^3 / 4096^3 bf16 TFLOP/s:
// w4r 1281-1299 / 1271-1280, w4d 1287-1299 / 1263-1269, w4 1281-1289 /
// 1203-1204; w4r also takes 3.5% fewer cycles at 8192^3 in the counters
// (half the L2 read requests of w4, L2 latency 268 against 323 cycles).
// lds stays selectable (tune cache, CJ_HIP_GEMM_TILE).
// CJ_HIP_GEMM_TILE=<name> overrides the choice (tuning sweeps), like the
// reference's CJ_* tuning variables.
enum class HalfTile { kW4, kW4D, kW4R, kW4H, kLds, kBig8, kBig4, kMid, kSmall };

inline int tiles_for(int M, int N, int b) { return ((M + b - 1) / b) * ((N + b - 1) / b); }

inline HalfTile pick_half_tile(int M, int N, bool padded) {
  if (const char* env = getenv("CJ_HIP_GEMM_TILE")) {
    const std::string v(env);
    if (v == "w4" && padded) return HalfTile::kW4;
    if (v == "w4d" && padded) return HalfTile::kW4D;
    if (v == "w4r" && padded) return HalfTile::kW4R;
    if (v == "w4h" && padded) return HalfTile::kW4H;
    if (v == "lds" && padded) return HalfTile::kLds;
    if (v == "big8") return HalfTile::kBig8;
    if (v == "big4") return HalfTile::kBig4;
    if (v == "mid") return HalfTile::kMid;
    if (v == "small") return HalfTile::kSmall;
  }
  constexpr int kCUs = 256;
  if (tiles_for(M, N, 256) >= kCUs) {
    return padded ? HalfTile::kW4H : HalfTile::kBig8;
  }
  if (tiles_for(M, N, 128) >= kCUs) {
    return HalfTile::kMid;
  }
  return HalfTile::kSmall;
}

template <typename T, int BM, int BN, int WM, int WN, typename LoadA, typename Epi, int STORE_AT = 32, int BK = kHBK>
static hipError_t launch_gemm_half_cfg(LoadA load_a, const uint16_t* Bt, int M, int N, int K, int ldb, Epi epi,
                                       hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_half_tn_kernel<T, BM, BN, BK, WM, WN, STORE_AT, LoadA, Epi>), dim3(tiles_m * tiles_n),
                     dim3(WM * WN * 64), 0, stream, load_a, Bt, M, N, K, ldb, tiles_n, epi);
  return hipGetLastError();
}

template <typename T, typename LoadA, typename Epi>
static hipError_t launch_gemm_half_tile(HalfTile tile, LoadA load_a, const uint16_t* Bt, int M, int N, int K,
                                        int ldb, Epi epi, hipStream_t stream) {
  switch (tile) {
    case HalfTile::kW4:
    case HalfTile::kW4D:
    case HalfTile::kW4R:
    case HalfTile::kW4H:
    case HalfTile::kLds:
    case HalfTile::kBig8:
      return launch_gemm_half_cfg<T, 256, 256, 2, 4>(load_a, Bt, M, N, K, ldb, epi, stream);
    case HalfTile::kBig4:
      // With four waves each holds a 128 x 128 block; the QKV epilogue's
      // address work on top of those 256 accumulators spills (1 KB per lane),
      // so a forced big4 runs that epilogue with eight waves.
      if constexpr (std::is_same_v<Epi, EpiQKV<T>>) {
        return launch_gemm_half_cfg<T, 256, 256, 2, 4>(load_a, Bt, M, N, K, ldb, epi, stream);
      } else {
        return launch_gemm_half_cfg<T, 256, 256, 2, 2>(load_a, Bt, M, N, K, ldb, epi, stream);
      }
    case HalfTile::kMid:
      return launch_gemm_half_cfg<T, 128, 128, 2, 2>(load_a, Bt, M, N, K, ldb, epi, stream);
    case HalfTile::kSmall:
    default:
      return launch_gemm_half_cfg<T, 64, 64, 2, 2>(load_a, Bt, M, N, K, ldb, epi, stream);
  }
}

template <typename T, typename LoadA, typename Epi>
static hipError_t launch_gemm_half(LoadA load_a, const uint16_t* Bt, int M, int N, int K, int ldb, Epi epi,
                                   hipStream_t stream) {
  return launch_gemm_half_tile<T>(pick_half_tile(M, N, false), load_a, Bt, M, N, K, ldb, epi, stream);
}

template <typename T, int BM, int BN, int WM, int WN, int NS, int BK = 64, typename ASrc, typename Epi>
static hipError_t launch_gemm_ring(ASrc asrc, const uint16_t* Bt, int M, int N, int K, int ldb, Epi epi,
                                   hipStream_t stream) {
  if (K % BK != 0) {
    return hipErrorInvalidValue;
  }
  const int tiles_n = (N + BN - 1) / BN;
  const dim3 grid(((M + BM - 1) / BM) * tiles_n);
  hipLaunchKernelGGL((gemm_half_ring_kernel<T, BM, BN, WM, WN, NS, ASrc, Epi, BK>), grid, dim3(WM * WN * 64), 0,
                     stream, asrc, Bt, M, N, K, ldb, tiles_n, epi);
  return hipGetLastError();
}

// The ring kernel serves the ViT GEMMs unless CJ_HIP_VIT_RING is 0 (A/B runs).
inline bool vit_ring_enabled() {
  const char* env = getenv("CJ_HIP_VIT_RING");
  return env == nullptr || std::string(env) != "0";
}

// 128-deep ring stages where K allows them, unless CJ_HIP_VIT_RING_BK is 64.
inline bool vit_ring_bk128(long long K) {
  const char* env = getenv("CJ_HIP_VIT_RING_BK");
  return K % 128 == 0 && (env == nullptr || std::string(env) != "64");
}

// Its copies use 32-bit byte offsets from a stage base and 16-byte alignment.
inline bool ring_fits(long long rows, long long ld) { return rows * ld * 2 < (1LL << 31) && ld % 8 == 0; }

// W4: 0 = gemm_half_tn_w4_kernel, 1 = gemm_half_tn_w4d_kernel, 2 = gemm_half_tn_w4r_kernel,
// 3 = gemm_half_tn_w4h_kernel
template <typename T, int W4>
static hipError_t launch_gemm_w4(const uint16_t* A, const uint16_t* Bt, float* C, int M, int N, int K, int lda,
                                 int ldb, int ldc, hipStream_t stream) {
  const int tiles_n = (N + 255) / 256;
  const dim3 grid(((M + 255) / 256) * tiles_n);
  if constexpr (W4 == 3) {
    const int vec4 = (ldc % 4 == 0 && reinterpret_cast<uintptr_t>(C) % 16 == 0) ? 1 : 0;
    hipLaunchKernelGGL((gemm_half_tn_w4h_kernel<T, EpiF32>), grid, dim3(256), 0, stream, A, Bt, M, N, K, lda, ldb,
                       tiles_n, EpiF32{C, ldc, vec4});
  } else if constexpr (W4 == 2) {
    hipLaunchKernelGGL((gemm_half_tn_w4r_kernel<T, EpiF32>), grid, dim3(256), 0, stream, A, Bt, M, N, K, lda, ldb,
                       tiles_n, EpiF32{C, ldc});
  } else if constexpr (W4 == 1) {
    hipLaunchKernelGGL((gemm_half_tn_w4d_kernel<T, EpiF32>), grid, dim3(256), 0, stream, A, Bt, M, N, K, lda, ldb,
                       tiles_n, EpiF32{C, ldc});
  } else {
    hipLaunchKernelGGL((gemm_half_tn_w4_kernel<T, EpiF32>), grid, dim3(256), 0, stream, A, Bt, M, N, K, lda, ldb,
                       tiles_n, EpiF32{C, ldc});
  }
  return hipGetLastError();
}

template <typename T, int WM, int WN>
static hipError_t launch_gemm_lds(const uint16_t* A, const uint16_t* Bt, float* C, int M, int N, int K, int lda,
                                  int ldb, int ldc, hipStream_t stream) {
  const int tiles_n = (N + 255) / 256;
  const dim3 grid(((M + 255) / 256) * tiles_n);
  hipLaunchKernelGGL((gemm_half_tn_lds_kernel<T, WM, WN, EpiF32>), grid, dim3(WM * WN * 64), 0, stream, A, Bt, M, N,
                     K, lda, ldb, tiles_n, EpiF32{C, ldc});
  return hipGetLastError();
}

}  // namespace lchip::k

namespace lchip::kern {

using namespace lchip::k;

hipError_t gemmF32(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                   hipStream_t stream) {
  return launch_gemm_f32<false>(A, B, M, N, K, lda, ldb, EpiStoreF32{C, ldc}, stream);
}

GemmF32Variant gemmF32Choose(int M, int N, int max_groups) {
  const char* env = getenv("CJ_HIP_GEMM_F32");
  const std::string v = env != nullptr ? env : "";
  if (v == "dp") return GemmF32Variant::kDataParallel;
  if (v == "sk") return GemmF32Variant::kStreamK;
  if (v == "bk32") return GemmF32Variant::kDataParallelBK32;
  // Whole tiles per workgroup when they fill the CUs evenly (or there are
  // many of them); stream-K otherwise.
  const int tiles = ((M + 63) / 64) * ((N + 63) / 64);
  return (tiles % max_groups != 0 && tiles < 8 * max_groups) ? GemmF32Variant::kStreamK
                                                              : GemmF32Variant::kDataParallel;
}

hipError_t gemmF32Padded(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                         const StreamKSync& sync, int max_groups, GemmF32Variant variant, hipStream_t stream) {
  if (K <= 0 || K % kF32GemmBK != 0 || lda % 4 != 0 || ldb % 4 != 0 || M <= 0 || N <= 0 || max_groups <= 0) {
    return hipErrorInvalidValue;
  }
  if (64LL * lda * 4 >= (1LL << 31) || 64LL * ldb * 4 >= (1LL << 31)) {
    // beyond the LDS kernel's 32-bit lane offsets (64 rows of either operand)
    return launch_gemm_f32<false>(A, B, M, N, K, lda, ldb, EpiStoreF32{C, ldc}, stream);
  }
  const int tiles_m = (M + 63) / 64;
  const int tiles_n = (N + 63) / 64;
  if (variant == GemmF32Variant::kAuto) {
    variant = gemmF32Choose(M, N, max_groups);
  }
  const bool bk32 = variant == GemmF32Variant::kDataParallelBK32;
  const int bk = bk32 ? 32 : 64;
  const int nk = K / bk;
  const int tiles = tiles_m * tiles_n;
  const bool sk = variant == GemmF32Variant::kStreamK;
  const long long iters = static_cast<long long>(tiles) * nk;
  const int groups = sk ? static_cast<int>(iters < max_groups ? iters : max_groups) : tiles;
  const EpiStoreF32 epi{C, ldc};
  if (bk32) {
    hipLaunchKernelGGL((gemm_f32_lds_kernel<32, 4, 2, false, EpiStoreF32>), dim3(groups), dim3(512), 0, stream, A,
                       B, M, N, lda, ldb, tiles_m, tiles_n, nk, sync, epi, 0);
  } else if (sk) {
    // Two stages (80 KB of LDS): measured fastest on every shape tried
    // (1024^3 to 4096x4096x1024, stream-K and whole tiles): a shorter
    // prologue, and room for two workgroups per CU on large grids.
    // XCD-local ranges below two tiles per workgroup (measured: 1000x777x1030
    // 24.9 -> 23.8 us; with more tiles per workgroup an XCD's concurrent tiles
    // scatter over its range: 1500^3 71.6 -> 77.4 us, so the global order stays).
    const int xl = (groups % 8 == 0 && tiles >= 8 && tiles < 2 * groups) ? 1 : 0;
    hipLaunchKernelGGL((gemm_f32_lds_kernel<64, 2, 2, true, EpiStoreF32>), dim3(groups), dim3(512), 0, stream, A, B,
                       M, N, lda, ldb, tiles_m, tiles_n, nk, sync, epi, xl);
  } else {
    hipLaunchKernelGGL((gemm_f32_lds_kernel<64, 2, 2, false, EpiStoreF32>), dim3(groups), dim3(512), 0, stream, A, B,
                       M, N, lda, ldb, tiles_m, tiles_n, nk, sync, epi, 0);
  }
  return hipGetLastError();
}

hipError_t gemmF32ConvNchw(const float* cols, const float* Wt, float* out, int M, int N, int K, const float* bias,
                           int relu, int ohw, hipStream_t stream) {
  return launch_gemm_f32<true>(cols, Wt, M, N, K, K, K, EpiConvNchwF32{out, bias, relu, N, ohw}, stream);
}

GemmHalfVariant gemmHalfChoose(int M, int N) {
  if (M <= 16) {
    return GemmHalfVariant::kSkinny;
  }
  switch (pick_half_tile(M, N, true)) {
    case HalfTile::kW4: return GemmHalfVariant::kW4;
    case HalfTile::kW4D: return GemmHalfVariant::kW4D;
    case HalfTile::kW4R: return GemmHalfVariant::kW4R;
    case HalfTile::kW4H: return GemmHalfVariant::kW4H;
    case HalfTile::kLds: return GemmHalfVariant::kLds;
    case HalfTile::kBig8: return GemmHalfVariant::kBig8;
    case HalfTile::kBig4: return GemmHalfVariant::kBig4;
    case HalfTile::kMid: return GemmHalfVariant::kMid;
    default: return GemmHalfVariant::kSmall;
  }
}

int skinnySplits(int N, int K, int cus) {
  const int tiles = (N + 16 * kSkinnyNT - 1) / (16 * kSkinnyNT);
  const int kblocks = (K + kSkinnyKB - 1) / kSkinnyKB;
  // Column tiles for half the CUs or more stream Bt as fast as more
  // workgroups would (16x8192x8192: 128 workgroups unsplit 21.3 us, 256 with
  // two splits 22.0-22.3 us): no split-K and its partial round trip.  Fewer
  // tiles split k until the CUs are covered, keeping two k-blocks per split.
  if (2 * tiles >= std::max(cus, 1)) {
    return 1;
  }
  int splits = 1;
  while (splits < kSkinnyMaxSplits && tiles * splits < std::max(cus, 1) && kblocks / (splits * 2) >= 2) {
    splits *= 2;
  }
  return splits;
}

hipError_t gemmHalfTN(const uint16_t* A, const uint16_t* Bt, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                      Half t, GemmHalfVariant variant, hipStream_t stream, const SkinnyWork* skinny) {
  if (K % kHBK != 0) {
    return hipErrorInvalidValue;
  }
  if (variant == GemmHalfVariant::kAuto) {
    variant = gemmHalfChoose(M, N);
  }
  if (variant == GemmHalfVariant::kSkinny && M > 16) {
    return hipErrorInvalidValue;  // the skinny kernel holds at most 16 rows of A
  }
  // A and Bt come from the resident upload, padded to 256 rows; the copies'
  // 32-bit lane offsets reach 256 rows of either operand.
  if ((variant == GemmHalfVariant::kLds || variant == GemmHalfVariant::kW4 || variant == GemmHalfVariant::kW4D ||
       variant == GemmHalfVariant::kW4R || variant == GemmHalfVariant::kW4H) &&
      (256LL * lda * 2 >= (1LL << 31) || 256LL * ldb * 2 >= (1LL << 31))) {
    variant = GemmHalfVariant::kBig8;
  }
  if (variant == GemmHalfVariant::kW4 && K > 0) {
    return t == Half::kBF16 ? launch_gemm_w4<BF16, 0>(A, Bt, C, M, N, K, lda, ldb, ldc, stream)
                            : launch_gemm_w4<F16, 0>(A, Bt, C, M, N, K, lda, ldb, ldc, stream);
  }
  if (variant == GemmHalfVariant::kW4D && K > 0) {
    return t == Half::kBF16 ? launch_gemm_w4<BF16, 1>(A, Bt, C, M, N, K, lda, ldb, ldc, stream)
                            : launch_gemm_w4<F16, 1>(A, Bt, C, M, N, K, lda, ldb, ldc, stream);
  }
  if (variant == GemmHalfVariant::kW4H && K > 0) {
    return t == Half::kBF16 ? launch_gemm_w4<BF16, 3>(A, Bt, C, M, N, K, lda, ldb, ldc, stream)
                            : launch_gemm_w4<F16, 3>(A, Bt, C, M, N, K, lda, ldb, ldc, stream);
  }
  if (variant == GemmHalfVariant::kW4R && K > 0) {
    return t == Half::kBF16 ? launch_gemm_w4<BF16, 2>(A, Bt, C, M, N, K, lda, ldb, ldc, stream)
                            : launch_gemm_w4<F16, 2>(A, Bt, C, M, N, K, lda, ldb, ldc, stream);
  }
  if (variant == GemmHalfVariant::kLds && K > 0) {
    return t == Half::kBF16 ? launch_gemm_lds<BF16, 2, 4>(A, Bt, C, M, N, K, lda, ldb, ldc, stream)
                            : launch_gemm_lds<F16, 2, 4>(A, Bt, C, M, N, K, lda, ldb, ldc, stream);
  }
  if (variant == GemmHalfVariant::kSkinny) {
    // Bt must be readable up to roundup(N, 64) rows and A up to 16 rows
    // (callers pad both to 256); split-K needs the workspace.
    const int tiles = (N + 16 * kSkinnyNT - 1) / (16 * kSkinnyNT);
    int splits = 1;
    if (skinny != nullptr && skinny->part != nullptr && skinny->counters != nullptr && tiles <= skinny->max_tiles) {
      splits = skinnySplits(N, K, skinny->cus);
      splits = std::min(splits, skinny->max_splits);
    }
    const dim3 grid(tiles, splits);
    float* part = splits > 1 ? skinny->part : nullptr;
    int* counters = splits > 1 ? skinny->counters : nullptr;
    if (t == Half::kBF16) {
      hipLaunchKernelGGL((gemm_skinny_kernel<BF16, kSkinnyNT, kSkinnyWaves, kSkinnyStages>), grid,
                         dim3(kSkinnyWaves * 64), 0, stream, A, Bt, C, M, N, K, lda, ldb, ldc, part, counters);
    } else {
      hipLaunchKernelGGL((gemm_skinny_kernel<F16, kSkinnyNT, kSkinnyWaves, kSkinnyStages>), grid,
                         dim3(kSkinnyWaves * 64), 0, stream, A, Bt, C, M, N, K, lda, ldb, ldc, part, counters);
    }
    return hipGetLastError();
  }
  const LoadRowMajor la{A, lda};
  const HalfTile tile = variant == GemmHalfVariant::kBig4  ? HalfTile::kBig4
                        : variant == GemmHalfVariant::kMid ? HalfTile::kMid
                        : variant == GemmHalfVariant::kSmall ? HalfTile::kSmall
                                                             : HalfTile::kBig8;
  if (t == Half::kBF16) {
    return launch_gemm_half_tile<BF16>(tile, la, Bt, M, N, K, ldb, EpiF32{C, ldc}, stream);
  }
  return launch_gemm_half_tile<F16>(tile, la, Bt, M, N, K, ldb, EpiF32{C, ldc}, stream);
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
  if (vit_ring_enabled() && (P == 8 || P == 16 || P == 32 || P == 64) &&
      static_cast<long long>(B) * C * H * W * 2 < (1LL << 31) && ring_fits(128, K)) {
    // 128x64 tiles (8 waves of 32x32): 156 workgroups at B = 8, 43 flop per
    // copied byte; measured faster than 64x64 (300 workgroups, 32 flop/B).
    // A 128-deep stage is 128/P kernel rows of one channel (P | 128, 128 | P*P).
    const RingPatch ra{x, C, H, W, P, T_, gw};
    if (P >= 16 && vit_ring_bk128(K)) {
      if (t == Half::kBF16) {
        return launch_gemm_ring<BF16, 128, 64, 4, 2, 3, 128>(ra, Wt, M, E, K, K, EpiHalf<BF16>{tokens, E, 1}, stream);
      }
      return launch_gemm_ring<F16, 128, 64, 4, 2, 3, 128>(ra, Wt, M, E, K, K, EpiHalf<F16>{tokens, E, 1}, stream);
    }
    if (t == Half::kBF16) {
      return launch_gemm_ring<BF16, 128, 64, 4, 2, 4>(ra, Wt, M, E, K, K, EpiHalf<BF16>{tokens, E, 1}, stream);
    }
    return launch_gemm_ring<F16, 128, 64, 4, 2, 4>(ra, Wt, M, E, K, K, EpiHalf<F16>{tokens, E, 1}, stream);
  }
  const LoadPatch la{x, M, C, H, W, P, T_, gw};
  if (t == Half::kBF16) {
    return launch_gemm_half<BF16>(la, Wt, M, E, K, K, EpiHalf<BF16>{tokens, E, 1}, stream);
  }
  return launch_gemm_half<F16>(la, Wt, M, E, K, K, EpiHalf<F16>{tokens, E, 1}, stream);
}

hipError_t patchTokensGemm(const uint16_t* xp, const uint16_t* Wt, uint16_t* tokens, int M, int K, int E, Half t,
                           hipStream_t stream) {
  if (K % kHBK != 0) {
    return hipErrorInvalidValue;
  }
  if (vit_ring_enabled() && ring_fits(128, K)) {
    const RingRowMajor ra{xp, K};
    if (vit_ring_bk128(K)) {
      if (t == Half::kBF16) {
        return launch_gemm_ring<BF16, 128, 64, 4, 2, 3, 128>(ra, Wt, M, E, K, K, EpiHalf<BF16>{tokens, E, 1}, stream);
      }
      return launch_gemm_ring<F16, 128, 64, 4, 2, 3, 128>(ra, Wt, M, E, K, K, EpiHalf<F16>{tokens, E, 1}, stream);
    }
    if (t == Half::kBF16) {
      return launch_gemm_ring<BF16, 128, 64, 4, 2, 4>(ra, Wt, M, E, K, K, EpiHalf<BF16>{tokens, E, 1}, stream);
    }
    return launch_gemm_ring<F16, 128, 64, 4, 2, 4>(ra, Wt, M, E, K, K, EpiHalf<F16>{tokens, E, 1}, stream);
  }
  const LoadRowMajor la{xp, K};
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
  const int Dh = E / H;
  // The ring kernel's accumulator stores need whole 4-row groups per image.
  if (vit_ring_enabled() && ring_fits(128, E) && T_ % 4 == 0) {
    // 128x128 tiles (8 waves): 234 workgroups for the B = 8 block, one per
    // CU; measured faster than 64x64 tiles (900 workgroups).
    // 64-deep stages here: a 128-deep stage of this tile is 64 KiB, so only
    // two fit and one stage is in flight; in the block, where the tokens come
    // cold from the patch GEMM, that measured 13.2 against 12.9 us.
    const RingRowMajor ra{tokens, E};
    if (t == Half::kBF16) {
      return launch_gemm_ring<BF16, 128, 128, 2, 4, 4>(ra, Wqkv_t, M, 3 * E, E, E,
                                                       EpiQKV<BF16>{q, k, vt, T_, E, H, Dh, S_pad}, stream);
    }
    return launch_gemm_ring<F16, 128, 128, 2, 4, 4>(ra, Wqkv_t, M, 3 * E, E, E,
                                                    EpiQKV<F16>{q, k, vt, T_, E, H, Dh, S_pad}, stream);
  }
  const LoadRowMajor la{tokens, E};
  if (t == Half::kBF16) {
    return launch_gemm_half<BF16>(la, Wqkv_t, M, 3 * E, E, E, EpiQKV<BF16>{q, k, vt, T_, E, H, Dh, S_pad}, stream);
  }
  return launch_gemm_half<F16>(la, Wqkv_t, M, 3 * E, E, E, EpiQKV<F16>{q, k, vt, T_, E, H, Dh, S_pad}, stream);
}

hipError_t outProjectGemm(const uint16_t* attn, const uint16_t* Wo_t, float* out, int M, int E, Half t,
                          hipStream_t stream) {
  if (E % kHBK != 0) {
    return hipErrorInvalidValue;
  }
  if (vit_ring_enabled() && ring_fits(128, E)) {
    const RingRowMajor ra{attn, E};
    if (vit_ring_bk128(E)) {
      if (t == Half::kBF16) {
        return launch_gemm_ring<BF16, 128, 64, 4, 2, 3, 128>(ra, Wo_t, M, E, E, E, EpiF32{out, E}, stream);
      }
      return launch_gemm_ring<F16, 128, 64, 4, 2, 3, 128>(ra, Wo_t, M, E, E, E, EpiF32{out, E}, stream);
    }
    if (t == Half::kBF16) {
      return launch_gemm_ring<BF16, 128, 64, 4, 2, 4>(ra, Wo_t, M, E, E, E, EpiF32{out, E}, stream);
    }
    return launch_gemm_ring<F16, 128, 64, 4, 2, 4>(ra, Wo_t, M, E, E, E, EpiF32{out, E}, stream);
  }
  return gemmHalfTN(attn, Wo_t, out, M, E, E, E, E, E, t, GemmHalfVariant::kAuto, stream);
}

}  // namespace lchip::kern
