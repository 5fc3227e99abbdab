// Autoregressive decode with a KV cache for DecoderLM (no counterpart in the
// reference: its attention reads the keys through a reinterpretation of k's
// buffer, so a position's key is not its own and cannot be cached; the decode
// uses textbook keys, the `textbook` mode of the attention core, with every
// rounding step of the reference's chain kept).
//
// One step feeds B tokens (one per sequence) at position pos and produces the
// next B tokens.  M = B rows everywhere, so each Linear is a weight stream:
// a wave per output column reads the column's K-contiguous weight row once
// and keeps the B rows of its input in LDS.  The step position lives in
// device memory (state[0]) so one captured graph serves every step:
//   state[0] = pos: position of the tokens being fed
//   state[1] = step index into the generated-token buffer
// Cache layout: [layer][b][h][Lmax][hd] for K and for V, 16-byte rows of
// the head dimension contiguous.
#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {
namespace {

constexpr int kSplit = 256;  // keys per attention block

template <int DT> struct Chunk {
  typedef typename Store<DT>::T T;
  static constexpr int E = 16 / sizeof(T);  // elements per 16-byte chunk
  static __device__ __forceinline__ void dec(uint4 c, float v[E]) {
    if constexpr (DT == F32) {
      v[0] = __uint_as_float(c.x); v[1] = __uint_as_float(c.y); v[2] = __uint_as_float(c.z); v[3] = __uint_as_float(c.w);
    } else {
      const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = Store<DT>::dec(uint16_t(w[i] & 0xffffu));
        v[2 * i + 1] = Store<DT>::dec(uint16_t(w[i] >> 16));
      }
    }
  }
};

// token + position rows of the tokens fed at state[0], one rounding
// (the prefill's embedding_pos chain)
template <int DT>
__global__ void __launch_bounds__(256)
dec_embed_kernel(const int32_t *__restrict__ ids, const typename Store<DT>::T *__restrict__ tok,
                 const typename Store<DT>::T *__restrict__ pos_tab, const int *__restrict__ state,
                 typename Store<DT>::T *__restrict__ out, int B, int V, int D, int *__restrict__ err) {
  typedef Store<DT> S;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= B) return;
  const int t = ids[row], p = state[0];
  const bool ok = t >= 0 && t < V;
  if (!ok && lane == 0) atomicOr(err, 1);
  const typename S::T *src = tok + long(ok ? t : 0) * D, *prow = pos_tab + long(p) * D;
  for (int d = lane; d < D; d += 64) out[long(row) * D + d] = S::enc(S::dec(prow[d]) + (ok ? S::dec(src[d]) : 0.f));
}

// The Linear output chain for one value (reference rounding per op):
// round(acc), round(+bias), GELU x*round(sigmoid(round(x*c))) rounded, then
// round(resid + x).
template <int DT, int ACT, bool RESID>
__device__ __forceinline__ float linear_chain(float acc, float bias, float gelu_c, float resid) {
  typedef Store<DT> S;
  float v = S::round(S::round(acc) + bias);
  if constexpr (ACT == ACT_GELU) {
    const float t = S::round(sigmoidf_ref(S::round(v * gelu_c)));
    v = S::round(v * t);
  }
  if constexpr (RESID) v = S::round(resid + v);
  return v;
}

// y[m][n] = chain(sum_k xin[m][k] W[n][k]) for m < M, one wave per column n.
// LN: xin = LayerNorm(x) (the LayerNorm kernel's arithmetic, rounded to the
// dtype), computed by every block into LDS; otherwise xin = x copied there.
// QKV: columns [0,E) go to q [M, E], [E,2E) and [2E,3E) to the K and V
// caches at position state[0] (head h = e / hd, element e % hd).
struct DecLinArgs {
  const void *x, *w, *bias, *ln_w, *ln_b, *resid;
  void *out, *kc, *vc;
  const int *state;
  int M, N, K, E, H, hd, Lmax;
  float eps, gelu_c;
};

template <int DT, bool LN, int ACT, bool RESID, bool QKV>
__global__ void __launch_bounds__(256) dec_linear_kernel(DecLinArgs a) {
  typedef Store<DT> S;
  typedef typename S::T T;
  typedef Chunk<DT> C;
  extern __shared__ uint4 xs[];  // [M][K / C::E] chunks
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = a.K, KC = K / C::E, M = a.M;
  const T *x = static_cast<const T *>(a.x);
  T *xl = reinterpret_cast<T *>(xs);
  if constexpr (LN) {
    const T *g = static_cast<const T *>(a.ln_w), *bb = static_cast<const T *>(a.ln_b);
    for (int m = wave; m < M; m += 4) {
      const T *xr = x + long(m) * K;
      float sum = 0.f;
      for (int c = lane; c < K; c += 64) sum += S::dec(xr[c]);
      const float mean = wave_sum(sum) / float(K);
      float var = 0.f;
      for (int c = lane; c < K; c += 64) {
        const float d = S::dec(xr[c]) - mean;
        var += d * d;
      }
      var = wave_sum(var) / float(K);
      const float inv = 1.0f / sqrtf(var + a.eps);
      for (int c = lane; c < K; c += 64) xl[long(m) * K + c] = S::enc((S::dec(xr[c]) - mean) * inv * S::dec(g[c]) + S::dec(bb[c]));
    }
  } else {
    const uint4 *xc = static_cast<const uint4 *>(a.x);
    for (int i = tid; i < M * KC; i += 256) xs[i] = xc[i];
  }
  __syncthreads();

  const int n = blockIdx.x * 4 + wave;
  if (n >= a.N) return;
  const uint4 *wr = static_cast<const uint4 *>(a.w) + long(n) * KC;
  float acc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) acc[m] = 0.f;
  for (int c = lane; c < KC; c += 64) {
    float wv[C::E];
    C::dec(wr[c], wv);
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      if (m < M) {
        float xv[C::E];
        C::dec(xs[m * KC + c], xv);
#pragma unroll
        for (int e = 0; e < C::E; ++e) acc[m] = fmaf(wv[e], xv[e], acc[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 16; ++m)
    if (m < M) acc[m] = wave_sum(acc[m]);
  // lane m finishes row m
  float mine = 0.f;
#pragma unroll
  for (int m = 0; m < 16; ++m)
    if (lane == m) mine = acc[m];
  if (lane >= M) return;
  const int m = lane;
  const float bias = a.bias ? S::dec(static_cast<const T *>(a.bias)[n]) : 0.f;
  const float res = RESID ? S::dec(static_cast<const T *>(a.resid)[long(m) * a.N + n]) : 0.f;
  const T y = S::enc(linear_chain<DT, ACT, RESID>(mine, bias, a.gelu_c, res));
  if constexpr (QKV) {
    const int which = n / a.E, e = n - which * a.E, h = e / a.hd, dd = e - h * a.hd;
    if (which == 0) {
      static_cast<T *>(a.out)[long(m) * a.E + e] = y;
    } else {
      T *cache = static_cast<T *>(which == 1 ? a.kc : a.vc);
      cache[((long(m) * a.H + h) * a.Lmax + a.state[0]) * a.hd + dd] = y;
    }
  } else {
    static_cast<T *>(a.out)[long(m) * a.N + n] = y;
  }
}

// Attention of the fed tokens over the cached keys 0..pos (all of them: the
// newest key is the query's own position).  Pass 1, one block per kSplit keys
// of head (b, h): score s_j = round(round(q.k_j) * scale) (the reference's
// matmul and scale roundings), kept in `scores`; the block's max and
// sum of exp(s_j - max) go to `stats`.
template <int DT>
__global__ void __launch_bounds__(kSplit)
dec_attn_scores_kernel(const typename Store<DT>::T *__restrict__ q, const typename Store<DT>::T *__restrict__ kc,
                       const int *__restrict__ state, float *__restrict__ scores, float2 *__restrict__ stats, int H,
                       int hd, int Lmax, float scale) {
  typedef Store<DT> S;
  typedef typename S::T T;
  typedef Chunk<DT> C;
  __shared__ float qs[256];
  __shared__ float red[kSplit / 64];
  const int s = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = bh / H, h = bh - b * H, L = state[0] + 1, nsplit = gridDim.x;
  for (int d = tid; d < hd; d += kSplit) qs[d] = S::dec(q[long(b) * H * hd + long(h) * hd + d]);
  __syncthreads();
  const int j = s * kSplit + tid;
  float sc = -INFINITY;
  if (j < L) {
    const uint4 *kr = reinterpret_cast<const uint4 *>(kc + (long(bh) * Lmax + j) * hd);
    float sum = 0.f;
    for (int c = 0; c < hd / C::E; ++c) {
      float kv[C::E];
      C::dec(kr[c], kv);
#pragma unroll
      for (int e = 0; e < C::E; ++e) sum = fmaf(qs[c * C::E + e], kv[e], sum);
    }
    sc = S::round(S::round(sum) * scale);
    scores[long(bh) * Lmax + j] = sc;
  }
  float mx = wave_max(sc);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < kSplit / 64; ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();
  float e = j < L ? __expf(sc - mx) : 0.f;
  e = wave_sum(e);
  if (lane == 0) red[wave] = e;
  __syncthreads();
  if (tid == 0) {
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < kSplit / 64; ++w) l += red[w];
    stats[long(bh) * nsplit + s] = make_float2(s * kSplit < L ? mx : -INFINITY, l);
  }
}

// Pass 2: the row's max M and sum S over every block's statistics (fixed
// order), probabilities p_j = round(exp(s_j - M) / S) like the reference's
// softmax output, then this block's share of sum_j p_j v_j (fp32) into
// `opart`.  The last block of the head to finish (a counter per head, reset
// by that block) adds the shares in block order and writes the rounded
// context.
template <int DT>
__global__ void __launch_bounds__(kSplit)
dec_attn_pv_kernel(const float *__restrict__ scores, const float2 *__restrict__ stats,
                   const typename Store<DT>::T *__restrict__ vc, const int *__restrict__ state,
                   float *__restrict__ opart, int *__restrict__ counters, typename Store<DT>::T *__restrict__ ctx, int H,
                   int hd, int Lmax) {
  typedef Store<DT> S;
  typedef typename S::T T;
  __shared__ float ps[kSplit];
  __shared__ float osh[16][65];
  __shared__ int last;
  const int s = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x, nsplit = gridDim.x;
  const int L = state[0] + 1;
  float Mx = -INFINITY;
  for (int i = 0; i < nsplit; ++i) Mx = fmaxf(Mx, stats[long(bh) * nsplit + i].x);
  float Ssum = 0.f;
  for (int i = 0; i < nsplit; ++i) {
    const float2 st = stats[long(bh) * nsplit + i];
    if (st.y > 0.f) Ssum += st.y * __expf(st.x - Mx);
  }
  const int j = s * kSplit + tid;
  ps[tid] = j < L ? S::round(__expf(scores[long(bh) * Lmax + j] - Mx) / Ssum) : 0.f;
  __syncthreads();
  // 16 key groups x 16 lanes of 4 head elements (hd <= 64)
  const int jg = tid >> 4, dq = (tid & 15) * 4;
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  if (dq < hd) {
    const int jn = min(kSplit, L - s * kSplit);
    for (int jj = jg; jj < jn; jj += 16) {
      float v[4];
      ld4<DT>(vc + (long(bh) * Lmax + s * kSplit + jj) * hd + dq, v);
      const float p = ps[jj];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = fmaf(p, v[e], o[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) osh[jg][(dq + e) & 63] = o[e];
  __syncthreads();
  if (tid < hd) {
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < 16; ++g) t += osh[g][tid];
    opart[(long(bh) * nsplit + s) * hd + tid] = t;
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) last = atomicAdd(&counters[bh], 1) == nsplit - 1;
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (tid < hd) {
    float t = 0.f;
    // device-coherent loads: the shares were written by other blocks
    for (int i = 0; i < nsplit; ++i)
      t += __int_as_float(__hip_atomic_load(reinterpret_cast<int *>(&opart[(long(bh) * nsplit + i) * hd + tid]),
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int b = bh / H, h = bh - b * H;
    ctx[long(b) * H * hd + long(h) * hd + tid] = S::enc(t);
  }
  if (tid == 0) atomicExch(&counters[bh], 0);
}

// Greedy choice: first index of each row's maximum (one block, waves split
// over the rows), written as the next step's input and into the generated
// tokens; then the position and the step index advance.
template <int DT>
__global__ void __launch_bounds__(1024)
dec_argmax_kernel(const typename Store<DT>::T *__restrict__ logits, int32_t *__restrict__ ids,
                  int32_t *__restrict__ tokens, int *__restrict__ state, int B, int V, int cap) {
  typedef Store<DT> S;
  __shared__ float bv[16];
  __shared__ int bi[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wpr = 16 / B;  // waves per row (B <= 16)
  const int row = wave / wpr, part = wave - row * wpr;
  float best = -INFINITY;
  int idx = 0x7fffffff;
  if (row < B) {
    const typename S::T *p = logits + long(row) * V;
    for (int c = part * 64 + lane; c < V; c += wpr * 64) {
      const float v = S::dec(p[c]);
      if (v > best || (idx == 0x7fffffff && v == best)) { best = v; idx = c; }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (ob > best || (ob == best && oi < idx)) { best = ob; idx = oi; }
  }
  if (lane == 0) { bv[wave] = best; bi[wave] = idx; }
  __syncthreads();
  if (tid < B) {
    float bb = -INFINITY;
    int ii = 0x7fffffff;
    for (int w = tid * wpr; w < (tid + 1) * wpr; ++w)
      if (bv[w] > bb || (bv[w] == bb && bi[w] < ii)) { bb = bv[w]; ii = bi[w]; }
    const int out = ii == 0x7fffffff ? 0 : ii;
    ids[tid] = out;
    const int st = state[1];
    if (st < cap) tokens[long(st) * B + tid] = out;
  }
  __syncthreads();
  if (tid == 0) {
    state[0] += 1;
    state[1] += 1;
  }
}

// Prefill: k / v [B*H, T, hd] into the caches' positions 0..T-1.
__global__ void __launch_bounds__(256)
kv_store_kernel(const uint4 *__restrict__ k, const uint4 *__restrict__ v, uint4 *__restrict__ kc,
                uint4 *__restrict__ vc, long rows, int T, int Lmax, int rc) {
  const long i = long(blockIdx.x) * 256 + threadIdx.x;  // chunk index
  if (i >= rows * rc) return;
  const long r = i / rc, c = i - r * rc;
  const long bh = r / T, t = r - bh * T;
  const long o = (bh * Lmax + t) * rc + c;
  kc[o] = k[i];
  vc[o] = v[i];
}

}  // namespace

hipError_t dec_embed(int dt, const int32_t *ids, const void *tok, const void *pos_tab, const int *state, void *out,
                     int B, int V, int D, int *err, hipStream_t st) {
  const dim3 grid((B + 3) / 4);
  switch (dt) {
  case F32: hipLaunchKernelGGL(dec_embed_kernel<F32>, grid, dim3(256), 0, st, ids, (const float *)tok, (const float *)pos_tab, state, (float *)out, B, V, D, err); break;
  case F16: hipLaunchKernelGGL(dec_embed_kernel<F16>, grid, dim3(256), 0, st, ids, (const uint16_t *)tok, (const uint16_t *)pos_tab, state, (uint16_t *)out, B, V, D, err); break;
  case BF16: hipLaunchKernelGGL(dec_embed_kernel<BF16>, grid, dim3(256), 0, st, ids, (const uint16_t *)tok, (const uint16_t *)pos_tab, state, (uint16_t *)out, B, V, D, err); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// kind: 0 LayerNorm + QKV, 1 + residual, 2 LayerNorm + GELU, 3 LayerNorm only
// (the head)
hipError_t dec_linear(int dt, int kind, const void *x, const void *w, const void *bias, const void *ln_w,
                      const void *ln_b, float eps, const void *resid, void *out, void *kc, void *vc, const int *state,
                      int M, int N, int K, int E, int H, int hd, int Lmax, float gelu_c, hipStream_t st) {
  const size_t es = dt_size(dt);
  if (M < 1 || M > 16 || K % int(16 / es) != 0 || size_t(M) * K * es > 65536) return hipErrorInvalidValue;
  DecLinArgs a{x, w, bias, ln_w, ln_b, resid, out, kc, vc, state, M, N, K, E, H, hd, Lmax, eps, gelu_c};
  const dim3 grid((N + 3) / 4);
  const size_t lds = size_t(M) * K * es;
#define MH_DL(DTV)                                                                                                     \
  switch (kind) {                                                                                                      \
  case 0: hipLaunchKernelGGL((dec_linear_kernel<DTV, true, ACT_NONE, false, true>), grid, dim3(256), lds, st, a); break;  \
  case 1: hipLaunchKernelGGL((dec_linear_kernel<DTV, false, ACT_NONE, true, false>), grid, dim3(256), lds, st, a); break; \
  case 2: hipLaunchKernelGGL((dec_linear_kernel<DTV, true, ACT_GELU, false, false>), grid, dim3(256), lds, st, a); break; \
  case 3: hipLaunchKernelGGL((dec_linear_kernel<DTV, true, ACT_NONE, false, false>), grid, dim3(256), lds, st, a); break; \
  default: return hipErrorInvalidValue;                                                                                \
  }
  switch (dt) {
  case F32: MH_DL(F32); break;
  case F16: MH_DL(F16); break;
  case BF16: MH_DL(BF16); break;
  default: return hipErrorInvalidValue;
  }
#undef MH_DL
  return hipGetLastError();
}

hipError_t dec_attention(int dt, const void *q, const void *kc, const void *vc, const int *state, float *scores,
                         float2 *stats, float *opart, int *counters, void *ctx, int B, int H, int hd, int Lmax,
                         float scale, hipStream_t st) {
  if (hd > 64 || hd % 4 != 0 || hd % int(16 / dt_size(dt)) != 0) return hipErrorInvalidValue;
  const dim3 grid((Lmax + kSplit - 1) / kSplit, B * H);
#define MH_DA(DTV, T)                                                                                               \
  hipLaunchKernelGGL(dec_attn_scores_kernel<DTV>, grid, dim3(kSplit), 0, st, (const T *)q, (const T *)kc, state,     \
                     scores, stats, H, hd, Lmax, scale);                                                             \
  hipLaunchKernelGGL(dec_attn_pv_kernel<DTV>, grid, dim3(kSplit), 0, st, scores, stats, (const T *)vc, state, opart, \
                     counters, (T *)ctx, H, hd, Lmax)
  switch (dt) {
  case F32: MH_DA(F32, float); break;
  case F16: MH_DA(F16, uint16_t); break;
  case BF16: MH_DA(BF16, uint16_t); break;
  default: return hipErrorInvalidValue;
  }
#undef MH_DA
  return hipGetLastError();
}

hipError_t dec_argmax(int dt, const void *logits, int32_t *ids, int32_t *tokens, int *state, int B, int V, int cap,
                      hipStream_t st) {
  if (B < 1 || B > 16) return hipErrorInvalidValue;
  switch (dt) {
  case F32: hipLaunchKernelGGL(dec_argmax_kernel<F32>, dim3(1), dim3(1024), 0, st, (const float *)logits, ids, tokens, state, B, V, cap); break;
  case F16: hipLaunchKernelGGL(dec_argmax_kernel<F16>, dim3(1), dim3(1024), 0, st, (const uint16_t *)logits, ids, tokens, state, B, V, cap); break;
  case BF16: hipLaunchKernelGGL(dec_argmax_kernel<BF16>, dim3(1), dim3(1024), 0, st, (const uint16_t *)logits, ids, tokens, state, B, V, cap); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t kv_store(int dt, const void *k, const void *v, void *kc, void *vc, int BH, int T, int hd, int Lmax,
                    hipStream_t st) {
  const int rc = int(size_t(hd) * dt_size(dt) / 16);
  if (size_t(hd) * dt_size(dt) % 16 != 0 || T > Lmax) return hipErrorInvalidValue;
  const long n = long(BH) * T * rc;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_store_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, (const uint4 *)k,
                     (const uint4 *)v, (uint4 *)kc, (uint4 *)vc, long(BH) * T, T, Lmax, rc);
  return hipGetLastError();
}

}  // namespace mh
