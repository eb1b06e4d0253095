// kernels.hpp -- host-side launchers for the gfx950 kernels.  Every launcher
// enqueues on the given stream and returns the launch status; shapes are
// validated by the callers (the dispatch layer) before launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace lchip::kern {

enum class Half { kBF16, kF16 };

// Tile geometry the callers pad buffers to.
constexpr int kHalfGemmBM = 256;  // rows of A a half-GEMM block may read
constexpr int kHalfGemmBN = 256;  // rows of Bt a half-GEMM block may read
constexpr int kHalfGemmBK = 64;   // K must be a multiple of this (zero-padded)
constexpr int kAttnQBlock = 128;  // queries per attention workgroup; S_pad multiple

constexpr int kF32GemmBM = 64;    // fp32 padded GEMM: rows of A a block reads
constexpr int kF32GemmBN = 64;    // columns of B a block reads
constexpr int kF32GemmBK = 64;    // K multiple (zero-padded)

// ---- fp32 ------------------------------------------------------------------
// C[M,N] = A[M,K] . B[K,N] (row-major, leading dimensions lda/ldb/ldc), any sizes.
hipError_t gemmF32(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                   hipStream_t stream);
// Workspace and protocol state of the stream-K fp32 GEMM.  `part` holds
// max_groups * 4096 floats of partial tiles and `flags` max_groups ints;
// a workgroup publishes its partial by storing `epoch` to its flag, and the
// owner clears the flags it saw set, so a launch without a timeout leaves
// every flag at zero.  The caller passes a new epoch per launch (flags start
// at zero; epochs from 1), so a flag a timed-out launch left set is never
// taken for ready later.  Owners poll a flag at most `spin_limit` times; one
// whose wait runs out stores 1 to *fail (device-visible memory the caller
// clears and checks after the stream sync) and that launch's result is
// invalid.  Launches that share part/flags must not overlap.
struct StreamKSync {
  float* part;
  int* flags;
  int* fail;
  int epoch;
  int spin_limit;
};
// Default bound of a stream-K owner's wait (polls of ~0.25 us each).
constexpr int kStreamKSpinLimit = 1 << 22;
// Same product on padded operands: A [roundup(M,64), K] (lda), B [K,
// roundup(N,64)] (ldb), K a multiple of kF32GemmBK, pads zero, lda/ldb
// multiples of 4 and both bases 16-byte aligned.  C [M, N] (ldc).  Stream-K
// over at most max_groups workgroups with the workspace in `sync`.
// Variants: whole 64x64 tiles per workgroup (BK 64 or 32), or stream-K
// (BK 64); kAuto takes CJ_HIP_GEMM_F32=dp|sk|bk32, else the heuristic of
// gemmF32Choose.
enum class GemmF32Variant { kAuto = 0, kDataParallel = 1, kStreamK = 2, kDataParallelBK32 = 3 };
GemmF32Variant gemmF32Choose(int M, int N, int max_groups);
hipError_t gemmF32Padded(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                         const StreamKSync& sync, int max_groups, GemmF32Variant variant, hipStream_t stream);
// dst[r][c] = src[r][c] (row stride ld_src) for r < rows, c < cols; 0 up to
// rows_pad x cols_pad (dst row stride cols_pad).
hipError_t padCopyF32(const float* src, float* dst, int rows, int cols, size_t ld_src, int rows_pad, int cols_pad,
                      hipStream_t stream);
// out2d = cols[M,K] . Wt^T where Wt is [N,K] (conv weights as stored, OIHW);
// epilogue adds bias, applies ReLU and scatters to NCHW out[img, n, pix]
// (m = img*ohw + pix).
hipError_t gemmF32ConvNchw(const float* cols, const float* Wt, float* out, int M, int N, int K, const float* bias,
                           int relu, int ohw, hipStream_t stream);
// cols[row, col] = x[n, c, oy*sh + ky - ph, ox*sw + kx - pw] (0 outside);
// row = (n*oh + oy)*ow + ox, col = (c*kh + ky)*kw + kx.
hipError_t im2colF32(const float* x, float* cols, int batch, int C, int H, int W, int kh, int kw, int sh, int sw,
                     int ph, int pw, int oh, int ow, hipStream_t stream);
// Up to four copies dst[0, n) = src[0, n) in one launch (either side may be the
// device alias of pinned host memory); with done_flag / done_count, the
// launch's completion flag as for attentionF32.
struct CopySegF32 {
  const float* src;
  float* dst;
  size_t n;
};
struct CopySegsF32 {
  CopySegF32 seg[4];
  int count;
};
hipError_t copySegsF32(const CopySegsF32& segs, hipStream_t stream, unsigned* done_count = nullptr,
                       unsigned* done_flag = nullptr, unsigned done_seq = 0);
// dst [0, n) = src [0, n), dst being the device alias of pinned host memory;
// then the launch's last workgroup writes done_seq to *done_flag (host-mapped)
// once every value is visible to the host, and leaves *done_count (device,
// zero) at zero.
hipError_t copyOutFlagF32(const float* src, float* dst, size_t n, unsigned* done_count, unsigned* done_flag,
                          unsigned done_seq, hipStream_t stream);
// Fills dst with the first `total` floats of the infinite repetition of src[0:n].
hipError_t repeatFillF32(const float* src, size_t n, float* dst, size_t total, hipStream_t stream);

// out[i] = a[i] (op) b[i] (b unused by kRelu); each element is read before it
// is written, so out may alias a or b.  kAddRelu also stores the sum before
// the ReLU to `sum` when that is not null.
enum class ElementwiseOp { kAdd = 0, kSub = 1, kDiv = 2, kRelu = 3, kAddRelu = 4 };
hipError_t elementwiseF32(ElementwiseOp op, const float* a, const float* b, float* out, float* sum, size_t n,
                          hipStream_t stream);

// x = relu?(x*scale + bias), in place (the attention output postprocess,
// reference src/attention.cpp:41-60).
hipError_t postprocessF32(float* x, size_t n, float scale, float bias, int relu, hipStream_t stream);

// Attention over `bh` independent [S, D] fp32 problems (head stride S*D),
// D <= 256.  Output postprocess relu?(o*post_scale + post_bias).  stats
// (optional, [bh, S, 2]) receives each query's softmax max m and sum l in the
// log2 domain (p = exp2((q.k)*scale*log2(e) - m) / l).
// With split_ws (device, split_ws_floats of it), a call whose 32-query grid
// would cover fewer than half the CUs divides the key tiles of each query
// block among workgroups that write partial results there; a second kernel
// merges them (attentionF32WorkspaceFloats: the floats such a call needs, 0
// when it would not split).
hipError_t attentionF32(const float* q, const float* k, const float* v, float* out, int bh, int S, int D,
                        bool causal, float post_scale, float post_bias, int post_relu, float* stats,
                        hipStream_t stream, int splits = 0, unsigned* done_count = nullptr,
                        unsigned* done_flag = nullptr, unsigned done_seq = 0, float* split_ws = nullptr,
                        size_t split_ws_floats = 0);
size_t attentionF32WorkspaceFloats(int bh, int S, int D, int splits);
// The `splits` value that selects the 16-query fp32 forward kernel
// (attn_fwd_f32_q16_kernel: 16 waves of 16-key tiles per 16 queries), for
// problems too small to fill the GPU.  Needs D <= 64, D % 4 == 0 and 16-byte
// aligned q / k / v; otherwise attentionF32 takes its heuristic split.
constexpr int kAttnF32Q16 = 16;
// attentionF32's choice for splits = 0: the 16-query kernel while its grid is
// at most one workgroup per CU (bh * S/16 <= 256, S <= 1024, D <= 64,
// D % 4 == 0), else the split heuristic below.
int attentionF32DefaultSplits(int bh, int S, int D);
// Key splits (waves per 32 queries) attentionF32 / attentionDvUpdateF32 use:
// `requested` (1, 2, 4 or 8) limited to what the head dim allows, or the
// heuristic when requested is 0.
int attentionF32Splits(int bh, int S, int D, int requested);
// The reference's conv -> attention chain in one launch: conv2d NCHW (+bias,
// ReLU) of x [batch, cin, h, wd] with w [cout, cin, kh, kw], Q/K/V = the
// consecutive S*D slices of its flat output repeated to 3*S*D values, then
// single-head non-causal attention -> out [S, D].  The conv output must have
// at most 8192 values.  With done_flag (host-mapped) and done_count (device,
// zero), the launch's last workgroup writes done_seq to *done_flag once every
// workgroup's output is visible to the host, and leaves the counter at zero
// (attentionF32 takes the same optional flag, without stats).
hipError_t convAttentionF32(const float* x, const float* w, const float* bias, int batch, int cin, int h, int wd,
                            int cout, int kh, int kw, int sh, int sw, int ph, int pw, int S, int D, float* out,
                            hipStream_t stream, unsigned* done_count = nullptr, unsigned* done_flag = nullptr,
                            unsigned done_seq = 0);
// True when convAttentionF32 reads x, w and bias exactly once per workgroup
// (all staged in LDS): then they may live in mapped host memory.
bool convAttentionStagesInputs(int batch, int cin, int h, int wd, int cout, int kh, int kw, int sh, int sw, int ph,
                               int pw);
// Train step backward: v -= lr * P^T . (2 (out - target) / (S*D)) per head,
// P recomputed from q, k and the forward's stats.
// With split_ws, small grids divide each key block's query tiles among
// workgroups writing partial dV there, summed and applied by a second kernel
// (attentionDvWorkspaceFloats: the floats such a call needs, 0 when it would
// not split).
hipError_t attentionDvUpdateF32(const float* q, const float* k, float* v, const float* out, const float* target,
                                const float* stats, int bh, int S, int D, bool causal, float lr,
                                hipStream_t stream, int splits = 0, float* split_ws = nullptr,
                                size_t split_ws_floats = 0);
size_t attentionDvWorkspaceFloats(int bh, int S, int D, int splits);
// *loss = norm * sum_i (out_i - target_i)^2 in a fixed order: contiguous
// chunks of 16384 elements per workgroup (at most kMseLossMaxBlocks), their
// partials added in chunk order by the last workgroup to finish.  partials
// holds kMseLossMaxBlocks floats and counter starts (and is left) at zero;
// without them one workgroup sums everything.
constexpr int kMseLossMaxBlocks = 64;
hipError_t mseLossF32(const float* out, const float* target, size_t n, float norm, float* loss, hipStream_t stream,
                      float* partials = nullptr, unsigned* counter = nullptr);

// ---- 16-bit ------------------------------------------------------------------
// dst[b][r][c] = half(src[b][r][c]) for r < rows, c < cols; 0 up to
// rows_pad x cols_pad.  src row stride ld_src, batch strides in elements.
hipError_t convertPad(const float* src, uint16_t* dst, int batch, int rows, int cols, size_t ld_src,
                      int rows_pad, int cols_pad, size_t src_bstride, size_t dst_bstride, Half t,
                      hipStream_t stream);
// ViT input: fp32 NCHW x -> 16-bit patch rows xp [B*T][C*P*P] (the im2col of
// the stride-P patch conv, a permutation of the image); P % 8 == 0, W % 8 == 0.
hipError_t vitPatchify(const float* x, uint16_t* xp, int B, int C, int H, int W, int P, Half t, hipStream_t stream);
// dst[b][c][r] = half(src[b][r][c]) (transpose), zero padding to
// cols_pad x rows_pad.
hipError_t convertTransposePad(const float* src, uint16_t* dst, int batch, int rows, int cols, size_t ld_src,
                               int rows_pad, int cols_pad, size_t src_bstride, size_t dst_bstride, Half t,
                               hipStream_t stream);

// C[M,N] (fp32, ldc) = A[M,K] . Bt[N,K]^T with A, Bt 16-bit row-major (lda,
// ldb), K a multiple of kHalfGemmBK, A readable up to roundup(M, 256) rows and
// Bt up to roundup(N, 256) rows.  Variants (block tile, waves): kW4 256x256
// with 4 waves and a ring of 32-deep k slices, kW4D the same waves over two
// 64-deep stages, kW4R / kW4H 4 waves over a ring of 64-deep parts (kW4H:
// barrier mid-stage, a half stage of fragments in registers, 16x16x32
// MFMAs), kLds 256x256 with 8 waves, all with direct
// global->LDS loads; kBig8 / kBig4 256x256 with 8 / 4 waves, kMid 128x128,
// kSmall 64x64, kSkinny for M <= 16 (split-K when given a SkinnyWork);
// kAuto follows gemmHalfChoose
// (CJ_HIP_GEMM_TILE=w4h|w4r|w4|w4d|lds|big8|big4|mid|small overrides it).
enum class GemmHalfVariant {
  kAuto = 0, kLds = 1, kBig8 = 2, kBig4 = 3, kMid = 4, kSmall = 5, kSkinny = 6, kW4 = 7, kW4D = 8, kW4R = 9,
  kW4H = 10
};
GemmHalfVariant gemmHalfChoose(int M, int N);
// Workspace of the skinny GEMM's split-K: partial tiles (max_splits x
// max_tiles x kSkinnyPartFloats floats) and one counter per column tile of
// 64 (zero at allocation; every launch leaves them at zero).  Launches that
// share it must not overlap.  cus: workgroups to aim for.
constexpr int kSkinnyMaxSplits = 8;
constexpr int kSkinnyPartFloats = 1024;  // one 16 x 64 fp32 partial
struct SkinnyWork {
  float* part;
  int* counters;
  int max_tiles;
  int max_splits;
  int cus;
};
// k-splits the skinny GEMM uses for N x K.
int skinnySplits(int N, int K, int cus);
hipError_t gemmHalfTN(const uint16_t* A, const uint16_t* Bt, float* C, int M, int N, int K, int lda, int ldb,
                      int ldc, Half t, GemmHalfVariant variant, hipStream_t stream,
                      const SkinnyWork* skinny = nullptr);
// Same GEMM with a 16-bit output (optionally ReLU).
hipError_t gemmHalfTNHalfOut(const uint16_t* A, const uint16_t* Bt, uint16_t* C, int M, int N, int K, int lda,
                             int ldb, int ldc, int relu, Half t, hipStream_t stream);

// Patch-embed convolution as implicit GEMM (kernel = stride = P, no padding):
// tokens[b*T + t, e] = relu(sum_k x[b, c, ty*P+ky, tx*P+kx] * w[e, c, ky, kx])
// with x 16-bit NCHW [B, C, H, W], Wt = w as [E, C*P*P] 16-bit; tokens 16-bit
// [roundup(B*T, 256), E].  Requires P % 8 == 0 and (C*P*P) % 64 == 0.
hipError_t patchEmbedGemm(const uint16_t* x, const uint16_t* Wt, uint16_t* tokens, int B, int C, int H, int W, int P,
                          int E, Half t, hipStream_t stream);
// The patch-embed conv as a row-major GEMM on vitPatchify's xp [M][K]:
// tokens = relu(xp . Wt^T), the same tiles and k order as patchEmbedGemm.
hipError_t patchTokensGemm(const uint16_t* xp, const uint16_t* Wt, uint16_t* tokens, int M, int K, int E, Half t,
                           hipStream_t stream);
// QKV projection for the ViT block: qkv = tokens[M, E] . Wqkv_t[3E, E]^T with
// the epilogue writing head-major Q, K [B*H, S_pad, Dh] and V transposed
// Vt [B*H, Dh, S_pad] (16-bit), M = B*T, S = T.
hipError_t qkvProjectGemm(const uint16_t* tokens, const uint16_t* Wqkv_t, uint16_t* q, uint16_t* k, uint16_t* vt,
                          int B, int T, int E, int H, int S_pad, Half t, hipStream_t stream);
// ViT output projection: out[M, E] (fp32) = attn[M, E] . Wo_t[E, E]^T (16-bit
// operands, E % 64 == 0).
hipError_t outProjectGemm(const uint16_t* attn, const uint16_t* Wo_t, float* out, int M, int E, Half t,
                          hipStream_t stream);

// Flash attention over `bh` problems: Q, K [bh, S_pad, D], Vt [bh, D, S_pad]
// (16-bit, zero padded to S_pad = roundup(S, 128)), D in {64, 128}.  Output
// either fp32 out_f32[bh, S, D] or, when out_heads_concat != nullptr, 16-bit
// rows out[(b*S + s), h*D + d] of a [B*S, H*D] matrix (heads = H).
hipError_t attentionHalf(const uint16_t* q, const uint16_t* k, const uint16_t* vt, float* out_f32,
                         uint16_t* out_heads_concat, int heads, int bh, int S, int S_pad, int D, bool causal, Half t,
                         hipStream_t stream);

// ViT: QKV projection of each (image, head) fused with its attention
// (vit_qkv_attn_kernel); tokens [B*T][E], Wqkv_t [3E][E], output
// heads-concatenated [B*T][E].  Needs E / H == 64, T <= 224 (the kernel's LDS
// holds 224 token rows), E % 64 == 0.
bool vitQkvAttentionFits(int T_, int E, int H);
hipError_t vitQkvAttention(const uint16_t* tokens, const uint16_t* Wqkv_t, uint16_t* out_heads_concat, int B,
                           int T_, int E, int H, Half t, hipStream_t stream);

}  // namespace lchip::kern
