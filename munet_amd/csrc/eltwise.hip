// Elementwise, gather and reduction-free kernels for gfx950.
//
// Reference semantics (all dtypes):
//   add/sub/mul/div with stride broadcasting ... BackendElementwiseCapability
//       (src/core/backend.hpp:207-217); strides come from compute_broadcast
//       (src/types.hpp:436-478) and address raw storage (view offsets are not
//       applied, src/core/ops/add.cpp:27-30).  fp32 computes in float
//       (src/backend/cpu_backend.hpp:238-332); fp16/bf16 compute the op on
//       the decoded values and round once (src/core/ops/common.hpp:46-85).
//   relu / sigmoid ............ src/backend/cpu_backend.hpp:493-531
//   exp/log/sqrt/rsqrt/sin/cos  src/backend/cpu_backend.hpp (unary family)
//   GELU ...................... nn::GELU, x * sigmoid(x * c) with c = 1.702
//       held in a [1] tensor of the dtype, three rounded ops
//       (src/nn/activations.hpp:31-38)
//   masked_fill ............... src/core/ops/elementwise.cpp:8-53
//   embedding gather .......... nn::Embedding index path
//       (src/nn/linear.hpp:92-128); out-of-range ids raise an error there,
//       here they write zeros and set a device error flag that the host
//       checks at its next synchronisation.
//   dtype conversion .......... Tensor::to(DataType) (src/tensor.cpp:249-284)
//       with the reference codecs.
//   argmax .................... first index of the row maximum (np.argmax as
//       used by demos/transformers/decoder_block_demo.py:112).
//
// Contiguous same-shape operands take a vectorised path (8 values per thread
// per step, 16-byte loads for 16-bit types); all kernels are grid-stride and
// sized to a few waves per CU.
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

__device__ __forceinline__ float binop(int op, float a, float b) {
  switch (op) {
  case BIN_ADD: return a + b;
  case BIN_SUB: return a - b;
  case BIN_MUL: return a * b;
  default: return a / b;
  }
}

template <int DT>
__global__ void binary_contig_kernel(const typename Store<DT>::T *__restrict__ a,
                                     const typename Store<DT>::T *__restrict__ b, typename Store<DT>::T *__restrict__ o,
                                     size_t n, int op) {
  typedef Store<DT> S;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    // reference fp32: float op; 16-bit: exact decoded op, single rounding
    o[i] = S::enc(binop(op, S::dec(a[i]), S::dec(b[i])));
  }
}

// 16-byte chunks: 8 values of a 16-bit type, 4 of fp32, decoded to floats
// and encoded back with the reference codecs.
template <int DT> struct Vec16 {
  typedef typename Store<DT>::T T;
  static constexpr int E = 16 / int(sizeof(T));
  static __device__ __forceinline__ void dec(uint4 q, float v[E]) {
    if constexpr (DT == F32) {
      v[0] = __uint_as_float(q.x); v[1] = __uint_as_float(q.y); v[2] = __uint_as_float(q.z); v[3] = __uint_as_float(q.w);
    } else {
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = Store<DT>::dec(uint16_t(w[i] & 0xffffu));
        v[2 * i + 1] = Store<DT>::dec(uint16_t(w[i] >> 16));
      }
    }
  }
  static __device__ __forceinline__ uint4 enc(const float v[E]) {
    if constexpr (DT == F32) {
      return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = uint32_t(Store<DT>::enc(v[2 * i])) | (uint32_t(Store<DT>::enc(v[2 * i + 1])) << 16);
      return make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
};

// Contiguous same-shape operands, whole 16-byte chunks (the host checks the
// alignment and n % E == 0): one chunk per thread per step, the op fixed at
// compile time.
template <int DT, int OP>
__global__ void __launch_bounds__(256) binary_vec_kernel(const uint4 *__restrict__ a, const uint4 *__restrict__ b,
                                                          uint4 *__restrict__ o, size_t chunks) {
  typedef Vec16<DT> V;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < chunks; i += stride) {
    float x[V::E], y[V::E];
    V::dec(a[i], x);
    V::dec(b[i], y);
#pragma unroll
    for (int e = 0; e < V::E; ++e) x[e] = binop(OP, x[e], y[e]);
    o[i] = V::enc(x);
  }
}

template <int DT>
__global__ void binary_bcast_kernel(const typename Store<DT>::T *__restrict__ a,
                                    const typename Store<DT>::T *__restrict__ b, typename Store<DT>::T *__restrict__ o,
                                    BcastArgs g, int op) {
  typedef Store<DT> S;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < g.total; i += stride) {
    size_t cur = i;
    long oa = 0, ob = 0;
    for (int d = g.ndim - 1; d >= 0; --d) {
      const size_t c = cur % size_t(g.shape[d]);
      cur /= size_t(g.shape[d]);
      oa += long(c) * g.sa[d];
      ob += long(c) * g.sb[d];
    }
    o[i] = S::enc(binop(op, S::dec(a[oa]), S::dec(b[ob])));
  }
}

// Row broadcast [rows, cols] op [cols] (bias add): no index division per
// element beyond one modulo.
template <int DT>
__global__ void binary_row_kernel(const typename Store<DT>::T *__restrict__ a,
                                  const typename Store<DT>::T *__restrict__ b, typename Store<DT>::T *__restrict__ o,
                                  size_t n, int cols, int op) {
  typedef Store<DT> S;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    o[i] = S::enc(binop(op, S::dec(a[i]), S::dec(b[i % cols])));
}

template <int DT>
__global__ void unary_kernel(const typename Store<DT>::T *__restrict__ in, typename Store<DT>::T *__restrict__ out,
                             size_t n, int op, float c) {
  typedef Store<DT> S;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float x = S::dec(in[i]);
    float y;
    switch (op) {
    case UN_RELU: y = x > 0.0f ? x : 0.0f; break;
    case UN_SIGMOID: y = sigmoidf_ref(x); break;
    case UN_GELU: {
      const float t1 = S::round(x * c);
      const float t2 = S::round(sigmoidf_ref(t1));
      y = x * t2;
      break;
    }
    case UN_EXP: y = __expf(x); break;
    case UN_LOG: y = __logf(x); break;
    case UN_SQRT: y = sqrtf(x); break;
    case UN_RSQRT: y = rsqrtf(x); break;
    case UN_SIN: y = sinf(x); break;
    default: y = cosf(x); break;
    }
    out[i] = S::enc(y);
  }
}

template <int DT, int OP>
__device__ __forceinline__ float unop(float x, float c) {
  typedef Store<DT> S;
  if constexpr (OP == UN_RELU) return x > 0.0f ? x : 0.0f;
  else if constexpr (OP == UN_SIGMOID) return sigmoidf_ref(x);
  else if constexpr (OP == UN_GELU) return x * S::round(sigmoidf_ref(S::round(x * c)));
  else if constexpr (OP == UN_EXP) return __expf(x);
  else if constexpr (OP == UN_LOG) return __logf(x);
  else if constexpr (OP == UN_SQRT) return sqrtf(x);
  else if constexpr (OP == UN_RSQRT) return rsqrtf(x);
  else if constexpr (OP == UN_SIN) return sinf(x);
  else return cosf(x);
}

// unary_kernel on whole 16-byte chunks, the op fixed at compile time
template <int DT, int OP>
__global__ void __launch_bounds__(256) unary_vec_kernel(const uint4 *__restrict__ in, uint4 *__restrict__ out,
                                                         size_t chunks, float c) {
  typedef Vec16<DT> V;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < chunks; i += stride) {
    float x[V::E];
    V::dec(in[i], x);
#pragma unroll
    for (int e = 0; e < V::E; ++e) x[e] = unop<DT, OP>(x[e], c);
    out[i] = V::enc(x);
  }
}

__global__ void masked_fill_kernel(const void *__restrict__ x, const int32_t *__restrict__ mask, void *__restrict__ out,
                                   size_t n, int dt, float value) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    st_any(out, dt, i, mask[i] != 0 ? value : ld_any(x, dt, i));
}

__global__ void convert_kernel(const void *__restrict__ in, int sdt, void *__restrict__ out, int ddt, size_t n) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    st_any(out, ddt, i, ld_any(in, sdt, i));
}

// One wave per token row; 16-bit rows of D values copied in 8-byte units.
// With `pos` set, adds the positional row (t = row % T) and rounds once, the
// fused form of token_embed(ids) + pos_embed(arange(T)).
template <int DT>
__global__ void __launch_bounds__(256)
embedding_kernel(const int32_t *__restrict__ ids, const typename Store<DT>::T *__restrict__ w,
                 const typename Store<DT>::T *__restrict__ pos, typename Store<DT>::T *__restrict__ out, int n, int V,
                 int D, int T, int *__restrict__ err) {
  typedef Store<DT> S;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const int tok = ids[row];
  const bool ok = tok >= 0 && tok < V;
  if (!ok && lane == 0) atomicOr(err, 1);
  const typename Store<DT>::T *src = w + long(ok ? tok : 0) * D;
  const typename Store<DT>::T *prow = pos ? pos + long(row % T) * D : nullptr;
  typename Store<DT>::T *dst = out + long(row) * D;
  for (int d = lane; d < D; d += 64) {
    float v = ok ? S::dec(src[d]) : 0.0f;
    if (prow) v = S::dec(prow[d]) + (ok ? v : 0.0f);
    dst[d] = S::enc(v);
  }
}

// Rows of D <= 256*NV values with D % 4 == 0: 4 values per lane per step,
// every load of the row issued before the first store.
template <int DT, int NV>
__global__ void __launch_bounds__(256)
embedding_vec_kernel(const int32_t *__restrict__ ids, const typename Store<DT>::T *__restrict__ w,
                     const typename Store<DT>::T *__restrict__ pos, typename Store<DT>::T *__restrict__ out, int n,
                     int V, int D, int T, int *__restrict__ err, float *__restrict__ stats) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const int tok = ids[row];
  const bool ok = tok >= 0 && tok < V;
  if (!ok && lane == 0) atomicOr(err, 1);
  const typename Store<DT>::T *src = w + long(ok ? tok : 0) * D;
  const typename Store<DT>::T *prow = pos ? pos + long(row % T) * D : nullptr;
  typename Store<DT>::T *dst = out + long(row) * D;
  float v[NV][4], p[NV][4];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = (k * 64 + lane) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[k][e] = p[k][e] = 0.f;
    if (c < D) {
      if (ok) ld4<DT>(src + c, v[k]);
      if (prow) ld4<DT>(prow + c, p[k]);
    }
  }
  // stats: the row's LayerNorm statistics over the stored (rounded) values,
  // (mean, M2) by two wave reductions
  float rsum = 0.f, r[NV][4];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = (k * 64 + lane) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[k][e] = 0.f;
    if (c < D) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = prow ? p[k][e] + v[k][e] : v[k][e];
      st4<DT>(dst + c, o);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r[k][e] = Store<DT>::round(o[e]);
        rsum += r[k][e];
      }
    }
  }
  if (stats) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) rsum += __shfl_xor(rsum, o, 64);
    const float mu = rsum / float(D);
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
      if ((k * 64 + lane) * 4 < D) {
#pragma unroll
        for (int e = 0; e < 4; ++e) q += (r[k][e] - mu) * (r[k][e] - mu);
      }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
    if (lane == 0) *reinterpret_cast<float2 *>(stats + 2 * long(row)) = make_float2(mu, q);
  }
}

// 16-bit rows of D <= 128*NC values, D % 8 == 0: one 16-lane DPP row of
// lanes per row (four rows per wave), NC 16-byte chunks per lane; the
// position row's loads go out beside the id's, the table row's once the id
// has arrived, and the statistics reduce within the DPP row (row16_sum).
template <int DT, int NC>
__global__ void __launch_bounds__(256)
embedding_row16_kernel(const int32_t *__restrict__ ids, const uint16_t *__restrict__ w,
                       const uint16_t *__restrict__ pos, uint16_t *__restrict__ out, int n, int V, int D, int T,
                       int *__restrict__ err, float *__restrict__ stats) {
  const int row = blockIdx.x * (blockDim.x >> 4) + (threadIdx.x >> 4);
  const int rl = threadIdx.x & 15;
  if (row >= n) return;  // the whole DPP row leaves together
  const int CH = D / 8;
  uint4 pq[NC], tq[NC];
  const uint4 *prow = pos ? reinterpret_cast<const uint4 *>(pos + long(row % T) * D) : nullptr;
  const int tok = ids[row];
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c = rl + 16 * k;
    pq[k] = prow && c < CH ? prow[c] : make_uint4(0, 0, 0, 0);
  }
  const bool ok = tok >= 0 && tok < V;
  if (!ok && rl == 0) atomicOr(err, 1);
  const uint4 *src = reinterpret_cast<const uint4 *>(w + long(ok ? tok : 0) * D);
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c = rl + 16 * k;
    tq[k] = ok && c < CH ? src[c] : make_uint4(0, 0, 0, 0);
  }
  uint4 *dst = reinterpret_cast<uint4 *>(out + long(row) * D);
  float r[NC][8];
  float rsum = 0.f;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int c = rl + 16 * k;
    float v[8], p[8];
    dec8<DT>(tq[k], v);
    dec8<DT>(pq[k], p);
#pragma unroll
    for (int e = 0; e < 8; ++e) r[k][e] = prow ? p[e] + v[e] : v[e];
    if (c < CH) {
      const uint4 o = enc8<DT>(r[k]);
      dst[c] = o;
      dec8<DT>(o, r[k]);  // the stored (rounded) values
#pragma unroll
      for (int e = 0; e < 8; ++e) rsum += r[k][e];
    }
  }
  if (stats) {
    // the row's LayerNorm statistics over the stored (rounded) values
    const float mu = row16_sum(rsum) / float(D);
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < NC; ++k)
      if (rl + 16 * k < CH)
#pragma unroll
        for (int e = 0; e < 8; ++e) q += (r[k][e] - mu) * (r[k][e] - mu);
    q = row16_sum(q);
    if (rl == 0) *reinterpret_cast<float2 *>(stats + 2 * long(row)) = make_float2(mu, q);
  }
}

// One wave per row: first index of the maximum (NaN never wins).
template <int DT>
__global__ void __launch_bounds__(256)
argmax_kernel(const typename Store<DT>::T *__restrict__ x, int32_t *__restrict__ out, int rows, int cols) {
  typedef Store<DT> S;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const typename Store<DT>::T *p = x + long(row) * cols;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int c = lane; c < cols; c += 64) {
    const float v = S::dec(p[c]);
    if (v > best || (bi == 0x7fffffff && v == best)) { best = v; bi = c; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
  }
  if (lane == 0) out[row] = bi == 0x7fffffff ? 0 : bi;
}

}  // namespace

hipError_t binary(int dt, int op, const void *a, const void *b, void *out, const BcastArgs &g, hipStream_t st) {
  if (g.total == 0) return hipSuccess;
  // classify: same contiguous shape, [rows, cols] + [cols], or general
  bool contig = true, row_bcast = g.ndim >= 1;
  long s = 1;
  for (int d = g.ndim - 1; d >= 0; --d) {
    if (g.sa[d] != s || g.sb[d] != s) contig = false;
    if (g.sa[d] != s) row_bcast = false;
    if (d == g.ndim - 1) { if (g.sb[d] != 1) row_bcast = false; }
    else if (g.sb[d] != 0) row_bcast = false;
    s *= g.shape[d];
  }
  const int blocks = grid_for(g.total, 256);
  const int cols = g.ndim ? g.shape[g.ndim - 1] : 1;
  const size_t per = dt == F32 ? 4 : 8;
  if (contig && g.total % per == 0 && (uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0 && (uintptr_t)out % 16 == 0 &&
      (dt == F32 || dt == F16 || dt == BF16)) {
    const size_t chunks = g.total / per;
    const int vb = grid_for(chunks, 256);
    const uint4 *a4 = static_cast<const uint4 *>(a), *b4 = static_cast<const uint4 *>(b);
    uint4 *o4 = static_cast<uint4 *>(out);
#define MH_BV(DTV, OPV) hipLaunchKernelGGL((binary_vec_kernel<DTV, OPV>), dim3(vb), dim3(256), 0, st, a4, b4, o4, chunks)
#define MH_BOP(DTV)                                                                                          \
  switch (op) {                                                                                              \
  case BIN_ADD: MH_BV(DTV, BIN_ADD); break;                                                                  \
  case BIN_SUB: MH_BV(DTV, BIN_SUB); break;                                                                  \
  case BIN_MUL: MH_BV(DTV, BIN_MUL); break;                                                                  \
  default: MH_BV(DTV, BIN_DIV); break;                                                                       \
  }
    if (dt == F32) { MH_BOP(F32) }
    else if (dt == F16) { MH_BOP(F16) }
    else { MH_BOP(BF16) }
#undef MH_BOP
#undef MH_BV
    return hipGetLastError();
  }
#define MH_BIN(DTV)                                                                                          \
  {                                                                                                          \
    typedef typename Store<DTV>::T T;                                                                        \
    if (contig)                                                                                              \
      hipLaunchKernelGGL(binary_contig_kernel<DTV>, dim3(blocks), dim3(256), 0, st, (const T *)a, (const T *)b, \
                         (T *)out, g.total, op);                                                             \
    else if (row_bcast)                                                                                      \
      hipLaunchKernelGGL(binary_row_kernel<DTV>, dim3(blocks), dim3(256), 0, st, (const T *)a, (const T *)b,    \
                         (T *)out, g.total, cols, op);                                                       \
    else                                                                                                     \
      hipLaunchKernelGGL(binary_bcast_kernel<DTV>, dim3(blocks), dim3(256), 0, st, (const T *)a, (const T *)b,  \
                         (T *)out, g, op);                                                                   \
  }
  switch (dt) {
  case F32: MH_BIN(F32); break;
  case F16: MH_BIN(F16); break;
  case BF16: MH_BIN(BF16); break;
  default: return hipErrorInvalidValue;
  }
#undef MH_BIN
  return hipGetLastError();
}

template <int DT>
void launch_unary_vec(int op, const void *in, void *out, size_t chunks, float c, hipStream_t st) {
  const int blocks = grid_for(chunks, 256);
  const uint4 *i4 = static_cast<const uint4 *>(in);
  uint4 *o4 = static_cast<uint4 *>(out);
#define MH_UN(OPV) hipLaunchKernelGGL((unary_vec_kernel<DT, OPV>), dim3(blocks), dim3(256), 0, st, i4, o4, chunks, c)
  switch (op) {
  case UN_RELU: MH_UN(UN_RELU); break;
  case UN_SIGMOID: MH_UN(UN_SIGMOID); break;
  case UN_GELU: MH_UN(UN_GELU); break;
  case UN_EXP: MH_UN(UN_EXP); break;
  case UN_LOG: MH_UN(UN_LOG); break;
  case UN_SQRT: MH_UN(UN_SQRT); break;
  case UN_RSQRT: MH_UN(UN_RSQRT); break;
  case UN_SIN: MH_UN(UN_SIN); break;
  default: MH_UN(UN_COS); break;
  }
#undef MH_UN
}

hipError_t unary(int dt, int op, const void *in, void *out, size_t n, float c, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const size_t per = dt == F32 ? 4 : 8;
  if (n % per == 0 && (uintptr_t)in % 16 == 0 && (uintptr_t)out % 16 == 0 && (dt == F32 || dt == F16 || dt == BF16)) {
    if (dt == F32) launch_unary_vec<F32>(op, in, out, n / per, c, st);
    else if (dt == F16) launch_unary_vec<F16>(op, in, out, n / per, c, st);
    else launch_unary_vec<BF16>(op, in, out, n / per, c, st);
    return hipGetLastError();
  }
  const int blocks = grid_for(n, 256);
  switch (dt) {
  case F32: hipLaunchKernelGGL(unary_kernel<F32>, dim3(blocks), dim3(256), 0, st, (const float *)in, (float *)out, n, op, c); break;
  case F16: hipLaunchKernelGGL(unary_kernel<F16>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)in, (uint16_t *)out, n, op, c); break;
  case BF16: hipLaunchKernelGGL(unary_kernel<BF16>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)in, (uint16_t *)out, n, op, c); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t masked_fill(int dt, const void *x, const int32_t *mask, void *out, size_t n, float value, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(masked_fill_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, x, mask, out, n, dt, value);
  return hipGetLastError();
}

// Every float bit pattern through the kernels' fp16 roundings (the
// branch-free one, and the four-wide one with its fast path) and through the
// full codec: counts the patterns where either differs in any bit.  Lane l
// of a wave takes patterns base + 4 l .. + 3, so a wave covers 256
// consecutive patterns per trip and fast-path and fallback waves both occur.
__global__ void __launch_bounds__(256) f16_round_check_kernel(unsigned long long *mismatches) {
  const uint32_t base = (blockIdx.x * 256u + (threadIdx.x >> 6) * 64u) * 256u + (threadIdx.x & 63u) * 4u;
  uint32_t bad = 0;
  for (uint32_t i = 0; i < 64u; ++i) {
    const uint32_t p0 = base + i * 256u;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(p0 + e);
    round4_f16(v);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = __uint_as_float(p0 + e);
      const uint32_t ref = __float_as_uint(round_f16_ref(x));
      bad += (__float_as_uint(v[e]) != ref) + (__float_as_uint(round_f16_exact(x)) != ref);
    }
  }
  if (bad) atomicAdd(mismatches, (unsigned long long)bad);
}

hipError_t check_f16_rounding(unsigned long long *mismatches, hipStream_t st) {
  unsigned long long *d = nullptr;
  hipError_t e = hipMalloc(&d, sizeof(*d));
  if (e != hipSuccess) return e;
  if ((e = hipMemsetAsync(d, 0, sizeof(*d), st)) == hipSuccess) {
    hipLaunchKernelGGL(f16_round_check_kernel, dim3(65536), dim3(256), 0, st, d);  // 2^32 patterns
    if ((e = hipGetLastError()) == hipSuccess &&
        (e = hipMemcpyAsync(mismatches, d, sizeof(*d), hipMemcpyDeviceToHost, st)) == hipSuccess)
      e = hipStreamSynchronize(st);
  }
  const hipError_t f = hipFree(d);
  return e != hipSuccess ? e : f;
}

hipError_t convert(int sdt, const void *in, int ddt, void *out, size_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(convert_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, in, sdt, out, ddt, n);
  return hipGetLastError();
}

hipError_t embedding(int dt, const int32_t *ids, const void *w, const void *pos, void *out, int n, int V, int D,
                     int T, int *err, hipStream_t st, float *stats) {
  if (n <= 0) return hipSuccess;
  dim3 grid((n + 3) / 4);
  const size_t es = dt == F32 ? 4 : 2;
  const bool vec = D % 4 == 0 && D <= 1024 && (uintptr_t)w % (4 * es) == 0 && (uintptr_t)out % (4 * es) == 0 &&
                   (uintptr_t)pos % (4 * es) == 0;
  if (stats && !vec) return hipErrorInvalidValue;  // LayerNorm statistics: vector path only
  if (dt != F32 && D % 8 == 0 && D <= 1024 && (uintptr_t)w % 16 == 0 && (uintptr_t)out % 16 == 0 &&
      (uintptr_t)pos % 16 == 0) {
    const dim3 g16((n + 3) / 4);  // one wave (four rows) per workgroup
    const uint16_t *W = (const uint16_t *)w, *P = (const uint16_t *)pos;
    uint16_t *O = (uint16_t *)out;
#define MH_EMB16(DTV, NC) \
  case NC: hipLaunchKernelGGL((embedding_row16_kernel<DTV, NC>), g16, dim3(64), 0, st, ids, W, P, O, n, V, D, T, err, stats); break
#define MH_EMB16_NC(DTV) \
  switch ((D / 8 + 15) / 16) { MH_EMB16(DTV, 1); MH_EMB16(DTV, 2); MH_EMB16(DTV, 3); MH_EMB16(DTV, 4); \
                               MH_EMB16(DTV, 5); MH_EMB16(DTV, 6); MH_EMB16(DTV, 7); MH_EMB16(DTV, 8); \
                               default: return hipErrorInvalidValue; }
    if (dt == F16) MH_EMB16_NC(F16) else MH_EMB16_NC(BF16)
#undef MH_EMB16_NC
#undef MH_EMB16
    return hipGetLastError();
  }
  if (vec) {
#define MH_EMB(DTV, T, NV)                                                                                      \
  hipLaunchKernelGGL((embedding_vec_kernel<DTV, NV>), grid, dim3(256), 0, st, ids, (const T *)w, (const T *)pos, \
                     (T *)out, n, V, D, T_, err, stats)
#define MH_EMB_NV(DTV, T) \
  { if (D <= 256) MH_EMB(DTV, T, 1); else if (D <= 512) MH_EMB(DTV, T, 2); else if (D <= 768) MH_EMB(DTV, T, 3); else MH_EMB(DTV, T, 4); }
    const int T_ = T;
    switch (dt) {
    case F32: MH_EMB_NV(F32, float); break;
    case F16: MH_EMB_NV(F16, uint16_t); break;
    case BF16: MH_EMB_NV(BF16, uint16_t); break;
    default: return hipErrorInvalidValue;
    }
#undef MH_EMB_NV
#undef MH_EMB
    return hipGetLastError();
  }
  switch (dt) {
  case F32: hipLaunchKernelGGL(embedding_kernel<F32>, grid, dim3(256), 0, st, ids, (const float *)w, (const float *)pos, (float *)out, n, V, D, T, err); break;
  case F16: hipLaunchKernelGGL(embedding_kernel<F16>, grid, dim3(256), 0, st, ids, (const uint16_t *)w, (const uint16_t *)pos, (uint16_t *)out, n, V, D, T, err); break;
  case BF16: hipLaunchKernelGGL(embedding_kernel<BF16>, grid, dim3(256), 0, st, ids, (const uint16_t *)w, (const uint16_t *)pos, (uint16_t *)out, n, V, D, T, err); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t argmax_rows(int dt, const void *x, int32_t *out, int rows, int cols, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  dim3 grid((rows + 3) / 4);
  switch (dt) {
  case F32: hipLaunchKernelGGL(argmax_kernel<F32>, grid, dim3(256), 0, st, (const float *)x, out, rows, cols); break;
  case F16: hipLaunchKernelGGL(argmax_kernel<F16>, grid, dim3(256), 0, st, (const uint16_t *)x, out, rows, cols); break;
  case BF16: hipLaunchKernelGGL(argmax_kernel<BF16>, grid, dim3(256), 0, st, (const uint16_t *)x, out, rows, cols); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mh
