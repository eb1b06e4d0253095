// convert.hip -- layout and precision passes that feed the MFMA kernels.
//
// These run once per upload (resident sessions) or once per one-shot call;
// they are HBM-bound streaming kernels: coalesced reads, 16-byte writes where
// the layout allows, and an LDS-staged 32x64 tile for the transposing form.
#include "../kernels.hpp"
#include "kcommon.hpp"

namespace lchip::k {

// ViT input: fp32 NCHW images -> 16-bit patch rows, xp[b*T + py*gw + px]
// [c*P*P + ky*P + kx] = x[b][c][py*P + ky][px*P + kx].  The im2col of an
// unpadded P x P conv with stride P is a permutation of the image, so the
// patch-embed conv becomes a row-major GEMM on xp.  One thread converts 8
// consecutive kx (two float4 loads, one 16-byte store); P % 8 == 0 and
// W % 8 == 0 keep every access aligned.
template <typename T>
__global__ __launch_bounds__(256) void patchify_kernel(const float* __restrict__ x, uint16_t* __restrict__ xp, int C,
                                                       int H, int W, int P, int gw, int T_, long long total8) {
  const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total8) {
    return;
  }
  const int K = C * P * P;
  const int k8 = K / 8;
  const long long m = i / k8;
  const int k = static_cast<int>(i - m * k8) * 8;
  const int b = static_cast<int>(m / T_);
  const int t = static_cast<int>(m - static_cast<long long>(b) * T_);
  const int py = t / gw;
  const int px = t - py * gw;
  const int c = k / (P * P);
  const int r = k - c * P * P;
  const int ky = r / P;
  const int kx = r - ky * P;
  const float* src = x + ((static_cast<size_t>(b) * C + c) * H + py * P + ky) * W + px * P + kx;
  const float4 lo = *reinterpret_cast<const float4*>(src);
  const float4 hi = *reinterpret_cast<const float4*>(src + 4);
  u32x4 o;
  o[0] = pack2<T>(lo.x, lo.y);
  o[1] = pack2<T>(lo.z, lo.w);
  o[2] = pack2<T>(hi.x, hi.y);
  o[3] = pack2<T>(hi.z, hi.w);
  *reinterpret_cast<u32x4*>(xp + m * K + k) = o;
}

template <typename T>
__global__ __launch_bounds__(256) void convert_pad_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                                          int rows, int cols, size_t ld_src, int rows_pad,
                                                          int cols_pad, size_t src_bstride, size_t dst_bstride) {
  const size_t b = blockIdx.z;
  src += b * src_bstride;
  dst += b * dst_bstride;
  // 4 output elements per thread along the (padded) row.
  const int c4 = (blockIdx.x * 256 + threadIdx.x) * 4;
  const int r = blockIdx.y;
  if (c4 >= cols_pad || r >= rows_pad) {
    return;
  }
  uint16_t h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = c4 + j;
    const float v = (r < rows && c < cols) ? src[static_cast<size_t>(r) * ld_src + c] : 0.0f;
    h[j] = to_half_bits<T>(v);
  }
  uint16_t* out = dst + static_cast<size_t>(r) * cols_pad + c4;
  if (c4 + 3 < cols_pad && (cols_pad & 3) == 0) {
    u32x2 w;
    w[0] = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
    w[1] = static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16);
    *reinterpret_cast<u32x2*>(out) = w;
  } else {
    for (int j = 0; j < 4 && c4 + j < cols_pad; ++j) {
      out[j] = h[j];
    }
  }
}

__global__ __launch_bounds__(256) void pad_copy_f32_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                           int rows, int cols, size_t ld_src, int rows_pad,
                                                           int cols_pad) {
  // 4 output elements per thread along the padded row; cols_pad % 4 == 0.
  const int c4 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c4 >= cols_pad) {
    return;
  }
  for (int r = blockIdx.y; r < rows_pad; r += gridDim.y) {
    float4 v;
    float* pv = reinterpret_cast<float*>(&v);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = c4 + j;
      pv[j] = (r < rows && c < cols) ? src[static_cast<size_t>(r) * ld_src + c] : 0.0f;
    }
    *reinterpret_cast<float4*>(dst + static_cast<size_t>(r) * cols_pad + c4) = v;
  }
}

// dst[c][r] = half(src[r][c]); block = 32 (r) x 64 (c) tile.
template <typename T>
__global__ __launch_bounds__(256) void convert_transpose_pad_kernel(const float* __restrict__ src,
                                                                    uint16_t* __restrict__ dst, int rows, int cols,
                                                                    size_t ld_src, int rows_pad, int cols_pad,
                                                                    size_t src_bstride, size_t dst_bstride) {
  __shared__ float tile[64][33];
  const size_t b = blockIdx.z;
  src += b * src_bstride;
  dst += b * dst_bstride;
  const int r0 = blockIdx.y * 32;
  const int c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63;
  const int ty = threadIdx.x >> 6;  // 0..3
  for (int rr = ty; rr < 32; rr += 4) {
    const int r = r0 + rr;
    const int c = c0 + tx;
    tile[tx][rr] = (r < rows && c < cols) ? src[static_cast<size_t>(r) * ld_src + c] : 0.0f;
  }
  __syncthreads();
  // write: dst row = c (64 of them), 32 consecutive r per row
  const int lr = threadIdx.x & 31;
  const int lc = threadIdx.x >> 5;  // 0..7
  for (int cc = lc; cc < 64; cc += 8) {
    const int c = c0 + cc;
    const int r = r0 + lr;
    if (c < cols_pad && r < rows_pad) {
      dst[static_cast<size_t>(c) * rows_pad + r] = to_half_bits<T>(tile[cc][lr]);
    }
  }
}

__global__ __launch_bounds__(256) void im2col_f32_kernel(const float* __restrict__ x, float* __restrict__ cols,
                                                         int C, int H, int W, int kh, int kw, int sh, int sw, int ph,
                                                         int pw, int oh, int ow, size_t total) {
  const int K = C * kh * kw;
  for (size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
       idx += static_cast<size_t>(gridDim.x) * 256) {
    const size_t row = idx / K;
    const int col = static_cast<int>(idx - row * K);
    const int c = col / (kh * kw);
    const int rr = col - c * kh * kw;
    const int ky = rr / kw;
    const int kx = rr - ky * kw;
    const int n = static_cast<int>(row / (static_cast<size_t>(oh) * ow));
    const int pix = static_cast<int>(row - static_cast<size_t>(n) * oh * ow);
    const int oy = pix / ow;
    const int ox = pix - oy * ow;
    const int y = oy * sh + ky - ph;
    const int xx = ox * sw + kx - pw;
    float v = 0.0f;
    if (y >= 0 && y < H && xx >= 0 && xx < W) {
      v = x[((static_cast<size_t>(n) * C + c) * H + y) * W + xx];
    }
    cols[idx] = v;
  }
}

__global__ __launch_bounds__(256) void repeat_fill_kernel(const float* __restrict__ src, size_t n,
                                                          float* __restrict__ dst, size_t total) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<size_t>(gridDim.x) * 256) {
    dst[i] = src[i % n];
  }
}

// Copies up to four (src, dst, n) segments in one launch: a small call's
// inputs out of mapped pinned staging (each value crosses the bus once), or
// its results into it.  Segment c runs as float4 when its n % 4 == 0 and both
// bases are 16-byte aligned.  With a completion flag, every wave releases its
// stores before the workgroup is counted.
__global__ __launch_bounds__(256) void copy_segs_f32_kernel(kern::CopySegsF32 segs, DoneFlag done) {
  const size_t stride = static_cast<size_t>(gridDim.x) * 256;
  const size_t first = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  for (int c = 0; c < segs.count; ++c) {
    const kern::CopySegF32 sg = segs.seg[c];
    const bool vec = sg.n % 4 == 0 && (reinterpret_cast<uintptr_t>(sg.src) | reinterpret_cast<uintptr_t>(sg.dst)) % 16 == 0;
    if (vec) {
      for (size_t i = first; i < sg.n / 4; i += stride) {
        reinterpret_cast<float4*>(sg.dst)[i] = reinterpret_cast<const float4*>(sg.src)[i];
      }
    } else {
      for (size_t i = first; i < sg.n; i += stride) {
        sg.dst[i] = sg.src[i];
      }
    }
  }
  done.finish_all_writers();
}

// out = a (op) b elementwise: 0 add, 1 sub, 2 div, 3 relu(a), 4 relu(a + b)
// (and a + b to `sum` when it is not null).
__global__ __launch_bounds__(256) void elementwise_f32_kernel(int op, const float* a, const float* b, float* out,
                                                              float* sum, size_t n) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * 256) {
    const float x = a[i];
    float v;
    switch (op) {
      case 0: v = x + b[i]; break;
      case 1: v = x - b[i]; break;
      case 2: v = x / b[i]; break;
      case 3: v = x < 0.0f ? 0.0f : x; break;
      default: {
        const float y = x + b[i];
        if (sum != nullptr) {
          sum[i] = y;
        }
        v = y < 0.0f ? 0.0f : y;
      }
    }
    out[i] = v;
  }
}

__global__ __launch_bounds__(256) void postprocess_kernel(float* __restrict__ x, size_t n, float scale, float bias,
                                                          int relu) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * 256) {
    float v = x[i] * scale + bias;
    if (relu && v < 0.0f) {
      v = 0.0f;
    }
    x[i] = v;
  }
}

}  // namespace lchip::k

namespace lchip::kern {

using namespace lchip::k;

static int grid_for(size_t total) {
  size_t blocks = (total + 255) / 256;
  if (blocks > 65536) {
    blocks = 65536;
  }
  return static_cast<int>(blocks < 1 ? 1 : blocks);
}

hipError_t convertPad(const float* src, uint16_t* dst, int batch, int rows, int cols, size_t ld_src, int rows_pad,
                      int cols_pad, size_t src_bstride, size_t dst_bstride, Half t, hipStream_t stream) {
  if (rows_pad <= 0 || cols_pad <= 0 || batch <= 0 || rows_pad > 65535) {
    return hipErrorInvalidValue;
  }
  const dim3 grid((cols_pad + 1023) / 1024, rows_pad, batch);
  if (t == Half::kBF16) {
    hipLaunchKernelGGL((convert_pad_kernel<BF16>), grid, dim3(256), 0, stream, src, dst, rows, cols, ld_src, rows_pad,
                       cols_pad, src_bstride, dst_bstride);
  } else {
    hipLaunchKernelGGL((convert_pad_kernel<F16>), grid, dim3(256), 0, stream, src, dst, rows, cols, ld_src, rows_pad,
                       cols_pad, src_bstride, dst_bstride);
  }
  return hipGetLastError();
}

hipError_t vitPatchify(const float* x, uint16_t* xp, int B, int C, int H, int W, int P, Half t, hipStream_t stream) {
  if (B <= 0 || C <= 0 || P <= 0 || P % 8 != 0 || W % 8 != 0 || H < P || W < P) {
    return hipErrorInvalidValue;
  }
  const int gh = H / P;
  const int gw = W / P;
  const int T_ = gh * gw;
  const long long total8 = static_cast<long long>(B) * T_ * C * P * P / 8;
  const dim3 grid(static_cast<unsigned>((total8 + 255) / 256));
  if (t == Half::kBF16) {
    hipLaunchKernelGGL((patchify_kernel<BF16>), grid, dim3(256), 0, stream, x, xp, C, H, W, P, gw, T_, total8);
  } else {
    hipLaunchKernelGGL((patchify_kernel<F16>), grid, dim3(256), 0, stream, x, xp, C, H, W, P, gw, T_, total8);
  }
  return hipGetLastError();
}

hipError_t padCopyF32(const float* src, float* dst, int rows, int cols, size_t ld_src, int rows_pad, int cols_pad,
                      hipStream_t stream) {
  if (rows_pad <= 0 || cols_pad <= 0 || cols_pad % 4 != 0 || rows > rows_pad || cols > cols_pad) {
    return hipErrorInvalidValue;
  }
  const dim3 grid((cols_pad + 1023) / 1024, rows_pad < 65535 ? rows_pad : 65535);
  hipLaunchKernelGGL(pad_copy_f32_kernel, grid, dim3(256), 0, stream, src, dst, rows, cols, ld_src, rows_pad,
                     cols_pad);
  return hipGetLastError();
}

hipError_t convertTransposePad(const float* src, uint16_t* dst, int batch, int rows, int cols, size_t ld_src,
                               int rows_pad, int cols_pad, size_t src_bstride, size_t dst_bstride, Half t,
                               hipStream_t stream) {
  if (rows_pad <= 0 || cols_pad <= 0 || batch <= 0) {
    return hipErrorInvalidValue;
  }
  const dim3 grid((cols_pad + 63) / 64, (rows_pad + 31) / 32, batch);
  if (t == Half::kBF16) {
    hipLaunchKernelGGL((convert_transpose_pad_kernel<BF16>), grid, dim3(256), 0, stream, src, dst, rows, cols, ld_src,
                       rows_pad, cols_pad, src_bstride, dst_bstride);
  } else {
    hipLaunchKernelGGL((convert_transpose_pad_kernel<F16>), grid, dim3(256), 0, stream, src, dst, rows, cols, ld_src,
                       rows_pad, cols_pad, src_bstride, dst_bstride);
  }
  return hipGetLastError();
}

hipError_t im2colF32(const float* x, float* cols, int batch, int C, int H, int W, int kh, int kw, int sh, int sw,
                     int ph, int pw, int oh, int ow, hipStream_t stream) {
  const size_t total = static_cast<size_t>(batch) * oh * ow * C * kh * kw;
  if (total == 0) {
    return hipSuccess;
  }
  hipLaunchKernelGGL(im2col_f32_kernel, dim3(grid_for(total)), dim3(256), 0, stream, x, cols, C, H, W, kh, kw, sh, sw,
                     ph, pw, oh, ow, total);
  return hipGetLastError();
}

hipError_t repeatFillF32(const float* src, size_t n, float* dst, size_t total, hipStream_t stream) {
  if (n == 0 || total == 0) {
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(repeat_fill_kernel, dim3(grid_for(total)), dim3(256), 0, stream, src, n, dst, total);
  return hipGetLastError();
}

hipError_t copySegsF32(const CopySegsF32& segs, hipStream_t stream, unsigned* done_count, unsigned* done_flag,
                       unsigned done_seq) {
  if (segs.count < 1 || segs.count > 4 || (done_flag != nullptr && done_count == nullptr)) {
    return hipErrorInvalidValue;
  }
  // Threads for the longest segment (float4 items where it vectorises), at
  // most 64 workgroups: with a flag, every workgroup is one more device-scope
  // count on the last one's path.
  size_t items = 0;
  for (int c = 0; c < segs.count; ++c) {
    const CopySegF32& sg = segs.seg[c];
    const bool vec = sg.n % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(sg.src) | reinterpret_cast<uintptr_t>(sg.dst)) % 16 == 0;
    const size_t w = vec ? sg.n / 4 : sg.n;
    items = w > items ? w : items;
  }
  if (items == 0) {
    return hipErrorInvalidValue;
  }
  const int grid = grid_for(items) < 64 ? grid_for(items) : 64;
  hipLaunchKernelGGL(copy_segs_f32_kernel, dim3(grid), dim3(256), 0, stream, segs,
                     DoneFlag{done_count, done_flag, done_seq});
  return hipGetLastError();
}

hipError_t copyOutFlagF32(const float* src, float* dst, size_t n, unsigned* done_count, unsigned* done_flag,
                          unsigned done_seq, hipStream_t stream) {
  if (n == 0 || done_count == nullptr || done_flag == nullptr) {
    return hipErrorInvalidValue;
  }
  CopySegsF32 segs{};
  segs.seg[0] = CopySegF32{src, dst, n};
  segs.count = 1;
  return copySegsF32(segs, stream, done_count, done_flag, done_seq);
}

}  // namespace lchip::kern

namespace lchip::kern {

hipError_t elementwiseF32(ElementwiseOp op, const float* a, const float* b, float* out, float* sum, size_t n,
                          hipStream_t stream) {
  if (n == 0) {
    return hipSuccess;
  }
  hipLaunchKernelGGL(elementwise_f32_kernel, dim3(grid_for(n)), dim3(256), 0, stream, static_cast<int>(op), a, b,
                     out, sum, n);
  return hipGetLastError();
}

hipError_t postprocessF32(float* x, size_t n, float scale, float bias, int relu, hipStream_t stream) {
  if (n == 0) {
    return hipSuccess;
  }
  hipLaunchKernelGGL(postprocess_kernel, dim3(grid_for(n)), dim3(256), 0, stream, x, n, scale, bias, relu);
  return hipGetLastError();
}

}  // namespace lchip::kern
