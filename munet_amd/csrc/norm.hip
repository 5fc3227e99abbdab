// Row-wise normalisation kernels for gfx950: LayerNorm and softmax.
//
// LayerNorm follows ops::layer_norm (src/core/ops/normalization.cpp:125-224):
// per row mean, biased variance, (x - mean) / sqrt(var + eps) * w + b, output
// rounded to the storage dtype.  The reference evaluates it in double on the
// host; here one wave (16-bit rows up to 1024 values: one 16-lane DPP row)
// owns a row, keeps it in registers, and reduces in fp32 across its lanes
// (two passes over registers, one HBM read and one HBM write per element).
//
// Softmax follows CPUBackend::softmax (src/backend/cpu_backend.hpp:587-611):
// float row max, double sum of exp(x - max), y = exp(x - max) / sum; the
// fp16/bf16 fallback (src/core/ops/activations.cpp:208-243) is the same
// arithmetic on decoded values with one rounding at the output.
#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {

namespace {

// VPL values per lane held in registers (row length <= 64*VPL).
template <int DT, int VPL>
__global__ void __launch_bounds__(256)
layernorm_kernel(const typename Store<DT>::T *__restrict__ x, const typename Store<DT>::T *__restrict__ w,
                 const typename Store<DT>::T *__restrict__ b, typename Store<DT>::T *__restrict__ y, int rows, int cols,
                 float eps) {
  typedef Store<DT> S;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const typename Store<DT>::T *xr = x + long(row) * cols;
  float v[VPL];
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int c = k * 64 + lane;
    v[k] = c < cols ? S::dec(xr[c]) : 0.f;
    sum += v[k];
  }
  const float mean = wave_sum(sum) / float(cols);
  float var = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int c = k * 64 + lane;
    const float d = c < cols ? v[k] - mean : 0.f;
    var += d * d;
  }
  var = wave_sum(var) / float(cols);
  const float inv = 1.0f / sqrtf(var + eps);
  typename Store<DT>::T *yr = y + long(row) * cols;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int c = k * 64 + lane;
    if (c < cols) yr[c] = S::enc((v[k] - mean) * inv * S::dec(w[c]) + S::dec(b[c]));
  }
}

// Rows of <= 256*NV values with cols % 4 == 0: each lane holds NV groups of 4
// consecutive values, every load of the row (x, w, b) is issued before the
// first reduction.
template <int DT, int NV>
__global__ void __launch_bounds__(256)
layernorm_vec_kernel(const typename Store<DT>::T *__restrict__ x, const typename Store<DT>::T *__restrict__ w,
                     const typename Store<DT>::T *__restrict__ b, typename Store<DT>::T *__restrict__ y, int rows,
                     int cols, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const typename Store<DT>::T *xr = x + long(row) * cols;
  float v[NV][4], wv[NV][4], bv[NV][4];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = (k * 64 + lane) * 4;
    if (c < cols) {
      ld4<DT>(xr + c, v[k]);
      ld4<DT>(w + c, wv[k]);
      ld4<DT>(b + c, bv[k]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[k][e] = wv[k][e] = bv[k][e] = 0.f;
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) sum += (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
  const float mean = wave_sum(sum) / float(cols);
  float var = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k)
    if ((k * 64 + lane) * 4 < cols)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[k][e] - mean;
        var += d * d;
      }
  var = wave_sum(var) / float(cols);
  const float inv = 1.0f / sqrtf(var + eps);
  typename Store<DT>::T *yr = y + long(row) * cols;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = (k * 64 + lane) * 4;
    if (c < cols) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (v[k][e] - mean) * inv * wv[k][e] + bv[k][e];
      st4<DT>(yr + c, o);
    }
  }
}

// 16-bit rows of cols <= 128*NC values, cols % 8 == 0: one 16-lane DPP row
// of lanes per row (four rows per wave), NC 16-byte chunks per lane, every
// load of the row (x, w, b) issued before the first reduction; the sums
// reduce within the DPP row (row16_sum), and the output leaves in 16-byte
// stores.
template <int DT, int NC>
__global__ void __launch_bounds__(256)
layernorm_row16_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ w, const uint16_t *__restrict__ b,
                       uint16_t *__restrict__ y, int rows, int cols, float eps) {
  const int row = blockIdx.x * (blockDim.x >> 4) + (threadIdx.x >> 4);
  const int rl = threadIdx.x & 15;
  if (row >= rows) return;  // the whole DPP row leaves together
  const int CH = cols / 8;
  const uint4 *xr = reinterpret_cast<const uint4 *>(x + long(row) * cols);
  const uint4 *wc = reinterpret_cast<const uint4 *>(w), *bc = reinterpret_cast<const uint4 *>(b);
  uint4 xq[NC], wq[NC], bq[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c = rl + 16 * k;
    const bool in = c < CH;
    xq[k] = in ? xr[c] : make_uint4(0, 0, 0, 0);
    wq[k] = in ? wc[c] : make_uint4(0, 0, 0, 0);
    bq[k] = in ? bc[c] : make_uint4(0, 0, 0, 0);
  }
  float v[NC][8];
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    dec8<DT>(xq[k], v[k]);
#pragma unroll
    for (int e = 0; e < 8; e += 2) sum += v[k][e] + v[k][e + 1];
  }
  const float mean = row16_sum(sum) / float(cols);
  float var = 0.f;
#pragma unroll
  for (int k = 0; k < NC; ++k)
    if (rl + 16 * k < CH)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[k][e] - mean;
        var += d * d;
      }
  var = row16_sum(var) / float(cols);
  const float inv = 1.0f / sqrtf(var + eps);
  uint4 *yr = reinterpret_cast<uint4 *>(y + long(row) * cols);
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c = rl + 16 * k;
    if (c < CH) {
      float wv[8], bv[8], o[8];
      dec8<DT>(wq[k], wv);
      dec8<DT>(bq[k], bv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (v[k][e] - mean) * inv * wv[e] + bv[e];
      yr[c] = enc8<DT>(o);
    }
  }
}

// Long rows: three streaming passes (mean, variance, normalise).
template <int DT>
__global__ void __launch_bounds__(256)
layernorm_long_kernel(const typename Store<DT>::T *__restrict__ x, const typename Store<DT>::T *__restrict__ w,
                      const typename Store<DT>::T *__restrict__ b, typename Store<DT>::T *__restrict__ y, int rows,
                      int cols, float eps) {
  typedef Store<DT> S;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const typename Store<DT>::T *xr = x + long(row) * cols;
  float sum = 0.f;
  for (int c = lane; c < cols; c += 64) sum += S::dec(xr[c]);
  const float mean = wave_sum(sum) / float(cols);
  float var = 0.f;
  for (int c = lane; c < cols; c += 64) {
    const float d = S::dec(xr[c]) - mean;
    var += d * d;
  }
  var = wave_sum(var) / float(cols);
  const float inv = 1.0f / sqrtf(var + eps);
  typename Store<DT>::T *yr = y + long(row) * cols;
  for (int c = lane; c < cols; c += 64) yr[c] = S::enc((S::dec(xr[c]) - mean) * inv * S::dec(w[c]) + S::dec(b[c]));
}

template <int DT>
__global__ void __launch_bounds__(256)
softmax_kernel(const typename Store<DT>::T *__restrict__ x, typename Store<DT>::T *__restrict__ y, int rows, int cols) {
  typedef Store<DT> S;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const typename Store<DT>::T *xr = x + long(row) * cols;
  float mx = -INFINITY;
  for (int c = lane; c < cols; c += 64) mx = fmaxf(mx, S::dec(xr[c]));
  mx = wave_max(mx);
  double sum = 0.0;
  for (int c = lane; c < cols; c += 64) sum += exp(double(S::dec(xr[c])) - double(mx));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  typename Store<DT>::T *yr = y + long(row) * cols;
  for (int c = lane; c < cols; c += 64) yr[c] = S::enc(float(exp(double(S::dec(xr[c])) - double(mx)) / sum));
}

template <int DT>
hipError_t ln_dt(const void *x, const void *w, const void *b, void *y, int rows, int cols, float eps, hipStream_t st) {
  typedef typename Store<DT>::T T;
  dim3 grid((rows + 3) / 4), block(256);
  const T *X = (const T *)x, *W = (const T *)w, *B = (const T *)b;
  T *Y = (T *)y;
  const bool vec = cols % 4 == 0 && (uintptr_t)x % (4 * sizeof(T)) == 0 && (uintptr_t)y % (4 * sizeof(T)) == 0 &&
                   (uintptr_t)w % (4 * sizeof(T)) == 0 && (uintptr_t)b % (4 * sizeof(T)) == 0;
  if constexpr (DT != F32) {
    const bool r16 = cols % 8 == 0 && cols <= 1024 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 &&
                     (uintptr_t)w % 16 == 0 && (uintptr_t)b % 16 == 0;
    if (r16) {
      // one wave (four rows) per workgroup: at 2048 rows of 512 (the
      // encoder block) 256-thread workgroups left half the CUs idle
      const dim3 g16((rows + 3) / 4);
      switch ((cols / 8 + 15) / 16) {
#define MH_LN16(NC) \
  case NC: hipLaunchKernelGGL((layernorm_row16_kernel<DT, NC>), g16, dim3(64), 0, st, X, W, B, Y, rows, cols, eps); break
        MH_LN16(1); MH_LN16(2); MH_LN16(3); MH_LN16(4); MH_LN16(5); MH_LN16(6); MH_LN16(7); MH_LN16(8);
#undef MH_LN16
      default: return hipErrorInvalidValue;
      }
      return hipGetLastError();
    }
  }
  if (vec && cols <= 256) hipLaunchKernelGGL((layernorm_vec_kernel<DT, 1>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  else if (vec && cols <= 512) hipLaunchKernelGGL((layernorm_vec_kernel<DT, 2>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  else if (vec && cols <= 768) hipLaunchKernelGGL((layernorm_vec_kernel<DT, 3>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  else if (vec && cols <= 1024) hipLaunchKernelGGL((layernorm_vec_kernel<DT, 4>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  else if (vec && cols <= 2048) hipLaunchKernelGGL((layernorm_vec_kernel<DT, 8>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  else if (cols <= 64 * 4) hipLaunchKernelGGL((layernorm_kernel<DT, 4>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  else if (cols <= 64 * 8) hipLaunchKernelGGL((layernorm_kernel<DT, 8>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  else if (cols <= 64 * 16) hipLaunchKernelGGL((layernorm_kernel<DT, 16>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  else hipLaunchKernelGGL((layernorm_long_kernel<DT>), grid, block, 0, st, X, W, B, Y, rows, cols, eps);
  return hipGetLastError();
}

}  // namespace

hipError_t layernorm(int dt, const void *x, const void *w, const void *b, void *y, int rows, int cols, float eps,
                     hipStream_t st) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  switch (dt) {
  case F32: return ln_dt<F32>(x, w, b, y, rows, cols, eps, st);
  case F16: return ln_dt<F16>(x, w, b, y, rows, cols, eps, st);
  case BF16: return ln_dt<BF16>(x, w, b, y, rows, cols, eps, st);
  default: return hipErrorInvalidValue;
  }
}

hipError_t softmax_rows(int dt, const void *x, void *y, int rows, int cols, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  dim3 grid((rows + 3) / 4), block(256);
  switch (dt) {
  case F32: hipLaunchKernelGGL(softmax_kernel<F32>, grid, block, 0, st, (const float *)x, (float *)y, rows, cols); break;
  case F16: hipLaunchKernelGGL(softmax_kernel<F16>, grid, block, 0, st, (const uint16_t *)x, (uint16_t *)y, rows, cols); break;
  case BF16: hipLaunchKernelGGL(softmax_kernel<BF16>, grid, block, 0, st, (const uint16_t *)x, (uint16_t *)y, rows, cols); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mh
