// Data-movement kernels for gfx950 (all bit-exact copies or max selections).
//
//   to_contiguous ...... BackendAllocationTransferCapability::to_contiguous
//                        (src/core/backend.hpp:202-204; CPU restatement of the
//                        strided gather in src/backend/cpu_backend.hpp:1139-1156)
//   transpose2d ........ [rows, cols] -> [cols, rows] per batch slice, used to
//                        feed transA/transB matmuls to the NT MFMA GEMM
//   concat ............. BackendShapeCapability::concat (backend.hpp:266-267,
//                        CPU copy in cpu_backend.hpp:416-452), any dim
//   max_pool2d ......... BackendSpatialCapability::max_pool2d, NCHW, window
//                        max with -1e9 initial value (cpu_backend.hpp:833-855)
//   upsample2d ......... nearest x scale, NCHW (src/core/ops/pooling.cpp:51-93)
//   NHWC variants ...... the same pooling / upsampling on the channels-last
//                        layout the conv engine path keeps resident
//   nchw <-> nhwc ...... layout change at the boundary of that path
// Tiled transposes stage 64x64 tiles through LDS so both the read and the
// write side are coalesced.
#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {

namespace {

inline int grid_for(size_t work, int per_block) {
  size_t g = (work + per_block - 1) / per_block;
  if (g > 256 * 16) g = 256 * 16;
  if (g < 1) g = 1;
  return int(g);
}

template <typename T>
__global__ void to_contig_kernel(const T *__restrict__ src, T *__restrict__ dst, StridedArgs g) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < g.total; i += stride) {
    size_t cur = i;
    long off = g.offset;
    for (int d = g.ndim - 1; d >= 0; --d) {
      const size_t c = cur % size_t(g.shape[d]);
      cur /= size_t(g.shape[d]);
      off += long(c) * g.strides[d];
    }
    dst[i] = src[off];
  }
}

template <typename T>
__global__ void __launch_bounds__(256)
transpose_kernel(const T *__restrict__ in, T *__restrict__ out, int rows, int cols) {
  __shared__ T tile[64][65];
  const long zoff = long(blockIdx.z) * rows * cols;
  in += zoff;
  out += zoff;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int gr = r0 + r, gc = c0 + tx;
    if (gr < rows && gc < cols) tile[r][tx] = in[long(gr) * cols + gc];
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int gc = c0 + c, gr = r0 + tx;
    if (gr < rows && gc < cols) out[long(gc) * rows + gr] = tile[tx][c];
  }
}

template <typename T>
__global__ void concat_kernel(const T *__restrict__ src, T *__restrict__ dst, size_t outer, size_t len, size_t out_len,
                              size_t off) {
  const size_t total = outer * len;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const size_t o = i / len, r = i - o * len;
    dst[o * out_len + off + r] = src[i];
  }
}

template <int DT>
__global__ void maxpool_nchw_kernel(const typename Store<DT>::T *__restrict__ in, typename Store<DT>::T *__restrict__ out,
                                    int B, int C, int iH, int iW, int k, int s, int p, int oH, int oW) {
  typedef Store<DT> S;
  const size_t total = size_t(B) * C * oH * oW;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int ow = int(idx % oW), oh = int((idx / oW) % oH);
    const size_t bc = idx / (size_t(oW) * oH);
    float mx = -1e9f;
    for (int kh = 0; kh < k; ++kh)
      for (int kw = 0; kw < k; ++kw) {
        const int ih = oh * s - p + kh, iw = ow * s - p + kw;
        if (ih >= 0 && ih < iH && iw >= 0 && iw < iW) mx = fmaxf(mx, S::dec(in[(bc * iH + ih) * iW + iw]));
      }
    out[idx] = S::enc(mx);
  }
}

template <int DT>
__global__ void maxpool_nhwc_kernel(const typename Store<DT>::T *__restrict__ in, typename Store<DT>::T *__restrict__ out,
                                    int B, int C, int iH, int iW, int k, int s, int p, int oH, int oW) {
  typedef Store<DT> S;
  const size_t total = size_t(B) * oH * oW * C;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int c = int(idx % C);
    const size_t pix = idx / C;
    const int ow = int(pix % oW), oh = int((pix / oW) % oH), b = int(pix / (size_t(oW) * oH));
    float mx = -1e9f;
    for (int kh = 0; kh < k; ++kh)
      for (int kw = 0; kw < k; ++kw) {
        const int ih = oh * s - p + kh, iw = ow * s - p + kw;
        if (ih >= 0 && ih < iH && iw >= 0 && iw < iW)
          mx = fmaxf(mx, S::dec(in[((size_t(b) * iH + ih) * iW + iw) * C + c]));
      }
    out[idx] = S::enc(mx);
  }
}

template <typename T>
__global__ void upsample_nchw_kernel(const T *__restrict__ in, T *__restrict__ out, int B, int C, int iH, int iW,
                                     int scale) {
  const int oH = iH * scale, oW = iW * scale;
  const size_t total = size_t(B) * C * oH * oW;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int ow = int(idx % oW), oh = int((idx / oW) % oH);
    const size_t bc = idx / (size_t(oW) * oH);
    out[idx] = in[(bc * iH + oh / scale) * iW + ow / scale];
  }
}

template <typename T>
__global__ void upsample_nhwc_kernel(const T *__restrict__ in, T *__restrict__ out, int B, int C, int iH, int iW,
                                     int scale) {
  const int oH = iH * scale, oW = iW * scale;
  const size_t total = size_t(B) * oH * oW * C;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total; idx += stride) {
    const int c = int(idx % C);
    const size_t pix = idx / C;
    const int ow = int(pix % oW), oh = int((pix / oW) % oH), b = int(pix / (size_t(oW) * oH));
    out[idx] = in[((size_t(b) * iH + oh / scale) * iW + ow / scale) * C + c];
  }
}

template <typename T>
hipError_t transpose_t(const void *in, void *out, int batch, int rows, int cols, hipStream_t st) {
  dim3 grid((cols + 63) / 64, (rows + 63) / 64, batch);
  hipLaunchKernelGGL(transpose_kernel<T>, grid, dim3(256), 0, st, (const T *)in, (T *)out, rows, cols);
  return hipGetLastError();
}

}  // namespace

hipError_t to_contiguous(int dt, const void *src, void *dst, const StridedArgs &g, hipStream_t st) {
  if (g.total == 0) return hipSuccess;
  const int blocks = grid_for(g.total, 256);
  if (dtype_size(dt) == 2)
    hipLaunchKernelGGL(to_contig_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)src, (uint16_t *)dst, g);
  else
    hipLaunchKernelGGL(to_contig_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, (const uint32_t *)src, (uint32_t *)dst, g);
  return hipGetLastError();
}

hipError_t transpose2d(int dt, const void *in, void *out, int batch, int rows, int cols, hipStream_t st) {
  if (batch <= 0 || rows <= 0 || cols <= 0) return hipSuccess;
  return dtype_size(dt) == 2 ? transpose_t<uint16_t>(in, out, batch, rows, cols, st)
                             : transpose_t<uint32_t>(in, out, batch, rows, cols, st);
}

hipError_t concat_part(int dt, const void *src, void *dst, size_t outer, size_t len, size_t out_len, size_t off,
                       hipStream_t st) {
  if (outer * len == 0) return hipSuccess;
  const int blocks = grid_for(outer * len, 256);
  if (dtype_size(dt) == 2)
    hipLaunchKernelGGL(concat_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)src, (uint16_t *)dst, outer, len, out_len, off);
  else
    hipLaunchKernelGGL(concat_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, (const uint32_t *)src, (uint32_t *)dst, outer, len, out_len, off);
  return hipGetLastError();
}

hipError_t max_pool2d(int dt, int nhwc, const void *in, void *out, int B, int C, int iH, int iW, int k, int s, int p,
                      hipStream_t st) {
  const int oH = (iH + 2 * p - k) / s + 1, oW = (iW + 2 * p - k) / s + 1;
  const size_t total = size_t(B) * C * oH * oW;
  if (total == 0) return hipSuccess;
  const int blocks = grid_for(total, 256);
#define MH_POOL(DTV)                                                                                                 \
  {                                                                                                                  \
    typedef typename Store<DTV>::T T;                                                                                \
    if (nhwc)                                                                                                        \
      hipLaunchKernelGGL(maxpool_nhwc_kernel<DTV>, dim3(blocks), dim3(256), 0, st, (const T *)in, (T *)out, B, C, iH, iW, k, s, p, oH, oW); \
    else                                                                                                             \
      hipLaunchKernelGGL(maxpool_nchw_kernel<DTV>, dim3(blocks), dim3(256), 0, st, (const T *)in, (T *)out, B, C, iH, iW, k, s, p, oH, oW); \
  }
  switch (dt) {
  case F32: MH_POOL(F32); break;
  case F16: MH_POOL(F16); break;
  case BF16: MH_POOL(BF16); break;
  default: return hipErrorInvalidValue;
  }
#undef MH_POOL
  return hipGetLastError();
}

hipError_t upsample2d(int dt, int nhwc, const void *in, void *out, int B, int C, int iH, int iW, int scale,
                      hipStream_t st) {
  const size_t total = size_t(B) * C * iH * iW * scale * scale;
  if (total == 0) return hipSuccess;
  const int blocks = grid_for(total, 256);
  if (dtype_size(dt) == 2) {
    if (nhwc) hipLaunchKernelGGL(upsample_nhwc_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)in, (uint16_t *)out, B, C, iH, iW, scale);
    else hipLaunchKernelGGL(upsample_nchw_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)in, (uint16_t *)out, B, C, iH, iW, scale);
  } else {
    if (nhwc) hipLaunchKernelGGL(upsample_nhwc_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, (const uint32_t *)in, (uint32_t *)out, B, C, iH, iW, scale);
    else hipLaunchKernelGGL(upsample_nchw_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, (const uint32_t *)in, (uint32_t *)out, B, C, iH, iW, scale);
  }
  return hipGetLastError();
}

// NCHW [B, C, HW] -> NHWC [B, HW, Cp] with channels C .. Cp-1 zero (the
// padded layout lets an implicit-GEMM convolution over few input channels
// take whole 16-byte chunks per pixel).
template <typename T>
__global__ void __launch_bounds__(256) nchw_to_nhwc_pad_kernel(const T *__restrict__ in, T *__restrict__ out, int C,
                                                               int HW, int Cp, size_t total) {
  for (size_t i = blockIdx.x * size_t(256) + threadIdx.x; i < total; i += size_t(gridDim.x) * 256) {
    const int c = int(i % Cp);
    const size_t pix = i / Cp, b = pix / HW, hw = pix - b * HW;
    out[i] = c < C ? in[(b * C + c) * HW + hw] : T(0);
  }
}

hipError_t nchw_to_nhwc_pad(int dt, const void *in, void *out, int B, int C, int HW, int Cp, hipStream_t st) {
  if (Cp < C) return hipErrorInvalidValue;
  const size_t total = size_t(B) * HW * Cp;
  if (total == 0) return hipSuccess;
  const int blocks = grid_for(total, 256);
  if (dtype_size(dt) == 2)
    hipLaunchKernelGGL(nchw_to_nhwc_pad_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)in,
                       (uint16_t *)out, C, HW, Cp, total);
  else
    hipLaunchKernelGGL(nchw_to_nhwc_pad_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, (const uint32_t *)in,
                       (uint32_t *)out, C, HW, Cp, total);
  return hipGetLastError();
}

// NCHW [B, C, HW] <-> NHWC [B, HW, C] is a batched 2-D transpose.
hipError_t nchw_to_nhwc(int dt, const void *in, void *out, int B, int C, int HW, hipStream_t st) {
  return transpose2d(dt, in, out, B, C, HW, st);
}
namespace {
// NHWC -> NCHW for a few channels (the UNet's 2-channel output): one thread
// per pixel reads its C contiguous values and writes each to its channel
// plane, so both the loads and every plane's stores are coalesced (a 64x64
// tile transpose would leave all but C of each tile's 64 columns idle).
template <typename T>
__global__ void __launch_bounds__(256) nhwc_to_nchw_fewc_kernel(const T *__restrict__ in, T *__restrict__ out, int C,
                                                                 long HW, long pixels) {
  const long stride = long(gridDim.x) * blockDim.x;
  for (long px = long(blockIdx.x) * blockDim.x + threadIdx.x; px < pixels; px += stride) {
    const long b = px / HW, hw = px - b * HW;
    const T *src = in + px * C;
    T *dst = out + b * C * HW + hw;
    for (int c = 0; c < C; ++c) dst[c * HW] = src[c];
  }
}
}  // namespace

hipError_t nhwc_to_nchw(int dt, const void *in, void *out, int B, int C, int HW, hipStream_t st) {
  if (C > 8) return transpose2d(dt, in, out, B, HW, C, st);
  const long pixels = long(B) * HW;
  if (pixels <= 0 || C <= 0) return hipSuccess;
  const int blocks = grid_for(size_t(pixels), 256);
  if (dtype_size(dt) == 2)
    hipLaunchKernelGGL(nhwc_to_nchw_fewc_kernel<uint16_t>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)in,
                       (uint16_t *)out, C, long(HW), pixels);
  else
    hipLaunchKernelGGL(nhwc_to_nchw_fewc_kernel<uint32_t>, dim3(blocks), dim3(256), 0, st, (const uint32_t *)in,
                       (uint32_t *)out, C, long(HW), pixels);
  return hipGetLastError();
}

}  // namespace mh
