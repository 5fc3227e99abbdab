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
// device memory (state[0]) so a captured graph serves every step (the host
// keeps one per count of 256-key attention blocks, 1..ceil(max_len / 256),
// and launches the one whose blocks hold keys 0..pos):
//   state[0] = pos: position of the tokens being fed
//   state[1] = step index into the generated-token buffer
//   state[2] = 1 while the head's greedy choices (best) are still to be fed
//              back: the next step's first kernel does it, or, after the
//              last step of a call, dec_finish_kernel
// Cache layout: [layer][b][h][Lmax][hd] for K and for V, 16-byte rows of
// the head dimension contiguous.
#include <type_traits>

#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {
namespace {

constexpr int kSplit = kDecKeyBlock;  // keys per attention block

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

// The step's first kernel.  The previous step's greedy choices, when pending
// (state[2], set by the head), become this step's input tokens and generated
// tokens: ids[b] and tokens[step][b], best reset, the position and the step
// index advanced.  Then the token + position rows of the fed tokens, one
// rounding (the prefill's embedding_pos chain), one thread per 16-byte chunk.
// One workgroup: every state read happens before its barrier and every state
// write after it, and the new position reaches the rows through LDS.
template <int DT>
__global__ void __launch_bounds__(256)
dec_embed_kernel(int32_t *__restrict__ ids, unsigned long long *__restrict__ best, int32_t *__restrict__ tokens,
                 int *__restrict__ state, const typename Store<DT>::T *__restrict__ tok,
                 const typename Store<DT>::T *__restrict__ pos_tab, typename Store<DT>::T *__restrict__ out, int B,
                 int V, int D, int cap, int *__restrict__ err) {
  typedef Chunk<DT> C;
  __shared__ int s_tok[16];
  __shared__ int s_pos;
  const int tid = threadIdx.x;
  const int p0 = state[0], st = state[1], pend = state[2];
  int t = 0;
  if (tid < B) {
    const unsigned long long k = best[tid];
    const int prev = ids[tid];
    t = pend ? (k ? int(0xffffffffu - uint32_t(k & 0xffffffffu)) : 0) : prev;
    s_tok[tid] = t;
  }
  if (tid == 0) s_pos = p0 + (pend ? 1 : 0);
  __syncthreads();
  if (pend) {
    if (tid < B) {
      ids[tid] = t;
      if (st < cap) tokens[long(st) * B + tid] = t;
      best[tid] = 0;
    }
    if (tid == 0) {
      state[0] = p0 + 1;
      state[1] = st + 1;
      state[2] = 0;
    }
  }
  const int p = s_pos, DC = D / C::E;
  for (int i = tid; i < B * DC; i += 256) {
    const int row = i / DC, cc = i - row * DC, tr = s_tok[row];
    const bool ok = tr >= 0 && tr < V;
    if (!ok && cc == 0) atomicOr(err, 1);
    const uint4 tv = reinterpret_cast<const uint4 *>(tok + long(ok ? tr : 0) * D)[cc];
    const uint4 pv = reinterpret_cast<const uint4 *>(pos_tab + long(p) * D)[cc];
    float a[C::E], pe[C::E];
    C::dec(tv, a);
    C::dec(pv, pe);
#pragma unroll
    for (int e = 0; e < C::E; ++e) a[e] = pe[e] + (ok ? a[e] : 0.f);
    reinterpret_cast<uint4 *>(out)[i] = C::enc(a);
  }
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

// Float -> unsigned key with the same order (NaN excluded by the caller);
// the argmax key is (key << 32) | ~index: the largest value, then the first
// index.  -0.0 takes +0.0's key: the two compare equal, so the first index
// of either must win, as in the prefill's argmax.
__device__ __forceinline__ uint32_t order_key(float v) {
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// acc + the dot product of two 16-byte chunks of 16-bit values (8 pairs), as
// four packed two-term dot products (v_dot2c_f32_bf16 / _f16: the products
// of 16-bit values are exact in fp32)
template <int DT> __device__ __forceinline__ float dot8(uint4 w, uint4 x, float acc) {
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w}, xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (DT == BF16) {
      typedef __bf16 b2 __attribute__((ext_vector_type(2)));
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, wv[j]), __builtin_bit_cast(b2, xv[j]), acc, false);
    } else {
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, wv[j]), __builtin_bit_cast(h2, xv[j]), acc, false);
    }
  }
  return acc;
}

// A 16-byte load with the non-temporal hint (the cached keys and values are
// read once per step and should not displace the weights in the caches).
__device__ __forceinline__ uint4 nt_load16(const uint4 *p) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// A zero chunk as a prvalue: `c ? p[i] : zero` with an lvalue zero is a
// glvalue conditional, compiled as a load through a selected address (a
// scratch copy of the zero, flat 4-byte loads) instead of a selected value.
__device__ __forceinline__ uint4 z4() { return make_uint4(0, 0, 0, 0); }

// Barrier that waits only for this wave's LDS operations: a __syncthreads()
// also waits for every outstanding global load, and those complete in issue
// order, so it would hold the input stage back until the last weight load
// of the block had arrived.
// The compiler fences keep LDS accesses on their side of the barrier (the
// two builtins alone do not order memory for the optimiser).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

enum DecIn : int { IN_ROW = 0, IN_LN = 1, IN_ATTN = 2 };
enum DecOut : int { OUT_ROW = 0, OUT_QKV = 1, OUT_ARGMAX = 2 };

// y[m][n] = chain(sum_k xin[m][k] W[n][k]) for M <= MB rows: each wave
// takes 4 output columns, one per 16-lane DPP row, and a column's
// K-contiguous weight row is split over its 16 lanes in 16-byte chunks
// (chunk c on lane c % 16, up to KCH per lane), so the dot products reduce
// with four DPP adds and no branch.  Each launch is a few
// microseconds of memory latency, so every global load a block needs is
// issued before the first wait: the input stage's loads first (its waits
// then cover only them), the weights next, the epilogue's bias and residual
// last.  Input stages:
//   IN_ROW : xin = x, copied to LDS;
//   IN_LN  : xin = LayerNorm(x) (fp32 mean and variance of the row, the
//            result rounded to the dtype, as the LayerNorm kernel), one row
//            per wave from registers;
//   IN_ATTN: xin = the attention context from dec_attn_kernel's per-block
//            shares: ctx = round(sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M)),
//            M the largest block max, in block order.
// Outputs: OUT_ROW y [M, N]; OUT_QKV columns [0,E) to q [M, E], [E,2E) and
// [2E,3E) to the K / V caches at position state[0]; OUT_ARGMAX y [M, N] and
// each row's greedy choice folded into best[m] by a 64-bit atomic max.
struct DecLinArgs {
  const void *x, *w, *bias, *ln_w, *ln_b, *resid;
  const float *part_o;
  const float2 *part_ml;
  void *out, *kc, *vc;
  unsigned long long *best;
  const int *state;
  int *pending;
  int M, N, K, E, H, hd, Lmax, nsplit;
  float eps, gelu_c;
};

constexpr int kMaxSplit = 16;  // key blocks per head (max_len <= 4096)

template <int DT, int KCH, int MB, int CPL, int WS, int IN, int OUT, int ACT, bool RESID>
__global__ void __launch_bounds__(256) dec_linear_kernel(DecLinArgs a) {
  typedef Store<DT> S;
  typedef typename S::T T;
  typedef Chunk<DT> C;
  static_assert(WS == 1 || WS == 4, "waves per column group");
  extern __shared__ uint4 xs[];  // [M][K / C::E] chunks of the staged input
  __shared__ unsigned long long bk[16 * CPL][16];
  __shared__ float wred[WS == 4 ? 4 : 1][4 * CPL][MB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = a.K, KC = K / C::E, M = a.M, N = a.N;
  constexpr int LCH = (KCH * WS + 3) / 4;  // LayerNorm: row chunks per lane (64 lanes)
  // column group of this wave (WS = 4: the four waves split one group's K)
  const int grp = WS == 1 ? wave : 0, q = WS == 1 ? 0 : wave;
  const int rl = lane & 15, row = lane >> 4;  // lane within its DPP row, row of the wave
  const int nbase = (blockIdx.x * (4 / WS) + grp) * 4 * CPL + row * CPL;  // this row's CPL columns

  // ---- 1. the input stage's loads
  constexpr int XR = 8;  // IN_ROW chunks per thread held in registers
  uint4 xq[IN == IN_ROW ? XR : 1];
  uint4 xr0[IN == IN_LN ? LCH : 1], gq[IN == IN_LN ? LCH : 1], bq[IN == IN_LN ? LCH : 1];
  if constexpr (IN == IN_ROW) {
    const uint4 *xc = static_cast<const uint4 *>(a.x);
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int i = tid + 256 * r;
      xq[r] = i < M * KC ? xc[i] : z4();
    }
  }
  // IN_ATTN with at most PS key blocks and at most PG groups of 4 context
  // values per thread: every share load is issued here, ahead of the
  // weights, instead of in trips of the input stage
  constexpr int PG = 3, PS = 4;
  float4 po[IN == IN_ATTN ? PG : 1][IN == IN_ATTN ? PS : 1];
  float2 pml[IN == IN_ATTN ? PG : 1][IN == IN_ATTN ? PS : 1];
  const int PG4 = M * K / 4;
  const bool pre = IN == IN_ATTN && a.nsplit <= PS && PG4 <= PG * 256;
  if constexpr (IN == IN_ATTN) {
    if (pre) {
      const int ns = a.nsplit;
#pragma unroll
      for (int u = 0; u < PG; ++u) {
        const int g = min(tid + 256 * u, PG4 - 1), e4 = g * 4, m = e4 / K, e = e4 - m * K, h = e / a.hd,
                  d = e - h * a.hd;
        const long bh = long(m) * a.H + h;
#pragma unroll
        for (int sp = 0; sp < PS; ++sp)
          if (sp < ns) {
            po[u][sp] = *reinterpret_cast<const float4 *>(a.part_o + (bh * ns + sp) * a.hd + d);
            pml[u][sp] = a.part_ml[bh * ns + sp];
          }
      }
    }
  }
  if constexpr (IN == IN_LN) {
    const uint4 *g = static_cast<const uint4 *>(a.ln_w), *bb = static_cast<const uint4 *>(a.ln_b);
    const uint4 *xr = static_cast<const uint4 *>(a.x) + long(min(wave, M - 1)) * KC;
#pragma unroll
    for (int i = 0; i < LCH; ++i) {
      const int c = lane + 64 * i;
      xr0[i] = c < KC ? xr[c] : z4();
      gq[i] = c < KC ? g[c] : z4();
      bq[i] = c < KC ? bb[c] : z4();
    }
  }

  // ---- 2. weights: chunks rl + 16 (q + WS i) of each of the row's columns
  // (loaded without a test: a load under a branch, even a wave-uniform one,
  // made the compiler's wait counts conservative, so that the input stage
  // waited for every weight load); the products use slots i < ni, the
  // chunk slots K needs
  const int ni = min(KCH, (KC + 16 * WS - 1) / (16 * WS));
  uint4 wv[CPL][KCH];
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc) {
    const uint4 *wr = static_cast<const uint4 *>(a.w) + long(min(nbase + cc, N - 1)) * KC;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = rl + 16 * (q + WS * i);
      wv[cc][i] = wr[min(c, KC - 1)];  // (chunks past K are never used)
    }
  }

  // ---- 3. the epilogue's operands (lane rl finishes row rl of its columns)
  // (kept raw: decoding them here would make the input stage wait for every
  // weight load issued before them)
  T braw[CPL], rraw[CPL];
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc) {
    const int nn = min(nbase + cc, N - 1), mm = min(rl, M - 1);
    braw[cc] = static_cast<const T *>(a.bias)[nn];
    rraw[cc] = RESID ? static_cast<const T *>(a.resid)[long(mm) * N + nn] : T(0);
  }
  // the cache position of the k / v stores (read here: loaded in the
  // epilogue it cost a memory round trip at the end of the kernel)
  const int kv_pos = OUT == OUT_QKV ? a.state[0] : 0;
  // every load above stays ahead of the input stage's arithmetic
  asm volatile("" ::: "memory");

  // ---- 4. stage the input in LDS
  if constexpr (IN == IN_ROW) {
    const uint4 *xc = static_cast<const uint4 *>(a.x);
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int i = tid + 256 * r;
      if (i < M * KC) xs[i] = xq[r];
    }
    for (int i = tid + 256 * XR; i < M * KC; i += 256) xs[i] = xc[i];
  } else if constexpr (IN == IN_LN) {
    for (int m = wave; m < M; m += 4) {
      float v[LCH][C::E];
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < LCH; ++i) {
        const int c = lane + 64 * i;
        C::dec(m == wave ? xr0[i] : (c < KC ? static_cast<const uint4 *>(a.x)[long(m) * KC + c] : z4()), v[i]);
#pragma unroll
        for (int e = 0; e < C::E; ++e) sum += v[i][e];
      }
      const float mean = wave_sum_dpp(sum) / float(K);
      float var = 0.f;
#pragma unroll
      for (int i = 0; i < LCH; ++i)
        if (lane + 64 * i < KC)
#pragma unroll
          for (int e = 0; e < C::E; ++e) {
            const float d = v[i][e] - mean;
            var += d * d;
          }
      var = wave_sum_dpp(var) / float(K);
      const float inv = 1.0f / sqrtf(var + a.eps);
#pragma unroll
      for (int i = 0; i < LCH; ++i) {
        const int c = lane + 64 * i;
        if (c < KC) {
          float gv[C::E], bv[C::E], o[C::E];
          C::dec(gq[i], gv);
          C::dec(bq[i], bv);
#pragma unroll
          for (int e = 0; e < C::E; ++e) o[e] = (v[i][e] - mean) * inv * gv[e] + bv[e];
          xs[m * KC + c] = C::enc(o);
        }
      }
    }
  } else {
    // groups of 4 consecutive context values of one head: from the shares
    // loaded up front, else two groups per trip with every share load of
    // both issued together
    T *xl = reinterpret_cast<T *>(xs);
    const int H = a.H, hd = a.hd, ns = a.nsplit, G4 = M * K / 4;
    if (pre) {
#pragma unroll
      for (int u = 0; u < PG; ++u) {
        const int g = tid + 256 * u;
        if (g < G4) {
          float mx = pml[u][0].x;
#pragma unroll
          for (int sp = 1; sp < PS; ++sp)
            if (sp < ns) mx = fmaxf(mx, pml[u][sp].x);
          float den = 0.f, num[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int sp = 0; sp < PS; ++sp)
            if (sp < ns && pml[u][sp].y > 0.f) {
              const float f = __expf(pml[u][sp].x - mx);
              den += pml[u][sp].y * f;
              num[0] += po[u][sp].x * f;
              num[1] += po[u][sp].y * f;
              num[2] += po[u][sp].z * f;
              num[3] += po[u][sp].w * f;
            }
          const float r = 1.0f / den;
#pragma unroll
          for (int e = 0; e < 4; ++e) xl[g * 4 + e] = S::enc(num[e] * r);
        }
      }
    }
    for (int g0 = pre ? G4 : tid; g0 < G4; g0 += 512) {
      float4 o[2][kMaxSplit];
      float2 ml[2][kMaxSplit];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int g = min(g0 + 256 * u, G4 - 1), e4 = g * 4, m = e4 / K, e = e4 - m * K, h = e / hd, d = e - h * hd;
        const long bh = long(m) * H + h;
#pragma unroll
        for (int sp = 0; sp < kMaxSplit; ++sp)
          if (sp < ns) {
            o[u][sp] = *reinterpret_cast<const float4 *>(a.part_o + (bh * ns + sp) * hd + d);
            ml[u][sp] = a.part_ml[bh * ns + sp];
          }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int g = g0 + 256 * u;
        if (g < G4) {
          float mx = ml[u][0].x;
#pragma unroll
          for (int sp = 1; sp < kMaxSplit; ++sp)
            if (sp < ns) mx = fmaxf(mx, ml[u][sp].x);
          float den = 0.f, num[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int sp = 0; sp < kMaxSplit; ++sp)
            if (sp < ns && ml[u][sp].y > 0.f) {
              const float f = __expf(ml[u][sp].x - mx);
              den += ml[u][sp].y * f;
              num[0] += o[u][sp].x * f;
              num[1] += o[u][sp].y * f;
              num[2] += o[u][sp].z * f;
              num[3] += o[u][sp].w * f;
            }
          const float r = 1.0f / den;
#pragma unroll
          for (int e = 0; e < 4; ++e) xl[g * 4 + e] = S::enc(num[e] * r);
        }
      }
    }
  }
  lds_barrier();

  // ---- 5. products, reductions, epilogue
  // Single-column products over up to 4 rows read every row's input chunks
  // before the first product: a chunk past K reads a clamped input chunk and
  // takes it as zeros (its weights are the clamped, finite chunk K - 1), rows
  // past M read row M - 1 and are never stored (a test per chunk and row put
  // each read in its own branch, followed by its own wait).  Up to 16 rows:
  // one row's chunks at a time, rows past M skipped by a wave-uniform test.
  float acc[CPL][MB];
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[cc][m] = 0.f;
  auto xload = [&](int i, int mm) -> uint4 {
    const int c = rl + 16 * (q + WS * i);
    const uint4 xv = xs[mm * KC + min(c, KC - 1)];
    return c < KC ? xv : z4();
  };
  auto prod = [&](int i, int m, uint4 x) {
    if constexpr (DT == F32) {
      float xv[C::E];
      C::dec(x, xv);
#pragma unroll
      for (int cc = 0; cc < CPL; ++cc) {
        float w[C::E];
        C::dec(wv[cc][i], w);
#pragma unroll
        for (int e = 0; e < C::E; ++e) acc[cc][m] = fmaf(w[e], xv[e], acc[cc][m]);
      }
    } else {
      // four packed dot products per chunk and row instead of 16 decodes and
      // 8 FMAs
#pragma unroll
      for (int cc = 0; cc < CPL; ++cc) acc[cc][m] = dot8<DT>(wv[cc][i], x, acc[cc][m]);
    }
  };
  if constexpr (MB == 4 && CPL == 1 && IN != IN_ATTN) {
    // every row's chunks read before the first product
    uint4 xr[MB][KCH];
#pragma unroll
    for (int i = 0; i < KCH; ++i)
      if (i < ni)
#pragma unroll
        for (int m = 0; m < MB; ++m) xr[m][i] = xload(i, min(m, M - 1));
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      if (i >= ni) break;
#pragma unroll
      for (int m = 0; m < MB; ++m) prod(i, m, xr[m][i]);
    }
  } else if constexpr (MB == 4) {
    // the vocabulary head (four columns per row: the batched reads above
    // would take it past 256 registers, one workgroup per CU) and the
    // out-projection (two of eight chunk slots used at d 768): one chunk at
    // a time, lanes past K idle
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = rl + 16 * (q + WS * i);
      if (c < KC) {
#pragma unroll
        for (int m = 0; m < MB; ++m)
          if (m < M) prod(i, m, xs[m * KC + c]);
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      if (m >= M) break;
      uint4 xr[KCH];
#pragma unroll
      for (int i = 0; i < KCH; ++i)
        if (i < ni) xr[i] = xload(i, m);
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        if (i >= ni) break;
        prod(i, m, xr[i]);
      }
    }
  }
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[cc][m] = row16_sum(acc[cc][m]);
  if constexpr (WS == 4) {
    // the four waves' shares of K, added in wave order by wave 0
    if (rl == 0) {
#pragma unroll
      for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
        for (int m = 0; m < MB; ++m) wred[q][row * CPL + cc][m] = acc[cc][m];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
      for (int m = 0; m < MB; ++m)
        acc[cc][m] = ((wred[0][row * CPL + cc][m] + wred[1][row * CPL + cc][m]) + wred[2][row * CPL + cc][m]) +
                     wred[3][row * CPL + cc][m];
  }

  unsigned long long key = 0;
#pragma unroll
  for (int cc = 0; cc < CPL; ++cc) {
    const int n = nbase + cc;
    float mine = acc[cc][0];
#pragma unroll
    for (int m = 1; m < MB; ++m)
      if (rl == m) mine = acc[cc][m];
    if (rl < M && n < N) {
      const int m = rl;
      const float bia = S::dec(braw[cc]), res = RESID ? S::dec(rraw[cc]) : 0.f;
      const T y = S::enc(linear_chain<DT, ACT, RESID>(mine, bia, a.gelu_c, res));
      if constexpr (OUT == OUT_QKV) {
        const int which = n / a.E, e = n - which * a.E, h = e / a.hd, dd = e - h * a.hd;
        if (which == 0) {
          static_cast<T *>(a.out)[long(m) * a.E + e] = y;
        } else {
          T *cache = static_cast<T *>(which == 1 ? a.kc : a.vc);
          cache[((long(m) * a.H + h) * a.Lmax + kv_pos) * a.hd + dd] = y;
        }
      } else {
        static_cast<T *>(a.out)[long(m) * N + n] = y;
      }
      if constexpr (OUT == OUT_ARGMAX) {
        const float yv = S::dec(y);
        if (yv == yv) {  // NaN never wins
          const unsigned long long k = (static_cast<unsigned long long>(order_key(yv)) << 32) | (0xffffffffu - uint32_t(n));
          key = k > key ? k : key;
        }
      }
    }
  }
  if constexpr (OUT == OUT_ARGMAX) {
    // row rl's best over the block's columns, then one atomic per row
    constexpr int SLOTS = (4 / WS) * 4;
    bk[grp * 4 + row][rl] = key;
    if constexpr (WS == 1) __syncthreads();
    else __builtin_amdgcn_s_waitcnt(0xc07f);  // wave 0 alone: its LDS writes done
    if (tid < M) {
      unsigned long long k = bk[0][tid];
#pragma unroll
      for (int c = 1; c < SLOTS; ++c) k = bk[c][tid] > k ? bk[c][tid] : k;
      if (k) atomicMax(&a.best[tid], k);
    }
    // the next kernel of the chain feeds the choices back
    if (blockIdx.x == 0 && tid == 0 && a.pending) *a.pending = 1;
  }
}

// Attention of the fed tokens over the cached keys 0..pos (the newest key is
// the query's own position), one block per kSplit keys of head (b, h), one
// wave per 64 of them, the way the prefill's flash kernel runs a key tile:
// scores s_j = round(round(q.k_j) * scale) (the reference's matmul and scale
// roundings), the wave's max m, p_j = round(e^(s_j - m)) (the rounded,
// unnormalised probabilities the product uses) and the wave's shares
// o = sum_j p_j v_j, l = sum_j p_j; the four waves' shares are rescaled to
// the block's max and added in wave order, into part_o / part_ml for the
// out-projection's input stage to combine.
// Lane layout: eight lanes per key row, lane c = lane & 7 holding dimensions
// 8c..8c+7 of rows (lane >> 3) + 8i, i = 0..7, of the wave's keys, so every
// K and V load instruction reads eight whole 128-byte rows (16-bit caches).
// Every K and V load of a thread is issued before the first wait.
template <int DT>
__global__ void __launch_bounds__(kSplit)
dec_attn_kernel(const typename Store<DT>::T *__restrict__ q, const typename Store<DT>::T *__restrict__ kc,
                const typename Store<DT>::T *__restrict__ vc, const int *__restrict__ state,
                float *__restrict__ part_o, float2 *__restrict__ part_ml, int H, int hd, int Lmax, float scale) {
  typedef Store<DT> S;
  typedef typename S::T T;
  constexpr int NU = int(sizeof(T)) / 2;  // 16-byte pieces per 8 dimensions
  constexpr int RW = 8;                   // key rows per lane
  __shared__ float wml[kSplit / 64][2];
  __shared__ float wo[kSplit / 64][4][64];
  const int s = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = bh / H, h = bh - b * H, ns = gridDim.x;
  const int c = lane & 7, rr = lane >> 3;
  const bool dim_ok = c * 8 < hd;
  const int cd = dim_ok ? c * 8 : 0;  // (lanes past hd load dimension 0 and are masked)
  const int jw = s * kSplit + wave * 64;  // the wave's first key
  // The position and q are loaded first; the K and V rows are clamped to the
  // position, so rows past it re-read the last cached row (cache hits)
  // instead of streaming rows 0..max_len-1 of every block, and a block past
  // the position leaves before loading any (an empty share).
  const int pos = state[0];
  uint4 qv[NU];
  {
    const uint4 *qp = reinterpret_cast<const uint4 *>(q + long(b) * H * hd + long(h) * hd + cd);
#pragma unroll
    for (int u = 0; u < NU; ++u) qv[u] = qp[u];
  }
  const int L = pos + 1;
  if (s * kSplit >= L) {
    if (tid < hd) part_o[(long(bh) * ns + s) * hd + tid] = 0.f;
    if (tid == 0) part_ml[long(bh) * ns + s] = make_float2(-INFINITY, 0.f);
    return;
  }
  const int jlast = min(pos, Lmax - 1);
  const T *kb = kc + long(bh) * Lmax * hd, *vb = vc + long(bh) * Lmax * hd;
  uint4 kr[RW][NU], vr[RW][NU];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const uint4 *kp = reinterpret_cast<const uint4 *>(kb + (min(jw + rr + 8 * i, jlast) * hd + cd));
#pragma unroll
    for (int u = 0; u < NU; ++u) kr[i][u] = nt_load16(kp + u);
  }
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const uint4 *vp = reinterpret_cast<const uint4 *>(vb + (min(jw + rr + 8 * i, jlast) * hd + cd));
#pragma unroll
    for (int u = 0; u < NU; ++u) vr[i][u] = nt_load16(vp + u);
  }
  // (every load above is issued before the first arithmetic that waits)
  __builtin_amdgcn_sched_barrier(0);

  // scores: each lane's 8-dimension partial, summed over the row's 8 lanes
  // (quad swaps, then the half-row mirror: every lane of the row ends with
  // the same sum)
  float qf[8];
  if constexpr (NU == 1) {
    dec8<DT>(qv[0], qf);
  } else {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      qf[4 * u] = __uint_as_float(qv[u].x); qf[4 * u + 1] = __uint_as_float(qv[u].y);
      qf[4 * u + 2] = __uint_as_float(qv[u].z); qf[4 * u + 3] = __uint_as_float(qv[u].w);
    }
  }
  float sc[RW];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    float part = 0.f;
    if constexpr (NU == 1) {
      part = dot8<DT>(kr[i][0], qv[0], 0.f);
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        part = fmaf(qf[4 * u], __uint_as_float(kr[i][u].x), part);
        part = fmaf(qf[4 * u + 1], __uint_as_float(kr[i][u].y), part);
        part = fmaf(qf[4 * u + 2], __uint_as_float(kr[i][u].z), part);
        part = fmaf(qf[4 * u + 3], __uint_as_float(kr[i][u].w), part);
      }
    }
    if (!dim_ok) part = 0.f;
    part += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(part), 0xb1, 0xf, 0xf, false));   // quad [1,0,3,2]
    part += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(part), 0x4e, 0xf, 0xf, false));   // quad [2,3,0,1]
    part += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(part), 0x141, 0xf, 0xf, false));  // half-row mirror
    const bool valid = jw + rr + 8 * i < L;
    sc[i] = valid ? S::round(S::round(part) * scale) : -INFINITY;
    mx = fmaxf(mx, sc[i]);
  }
  // the wave's max: the two row groups of a 16-lane DPP row (rotation by
  // 8), then the four DPP rows
  mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x128, 0xf, 0xf, false)));
  mx = rows4_max(mx);
  // masked keys (s = -inf) get p = e^-inf = 0, also in a wave with no key at
  // or before the position (mx = -inf, taken as 0)
  const float mxs = mx > -INFINITY ? mx : 0.f;
  float l = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const float p = S::round(__expf(sc[i] - mxs));
    l += p;
    float v[8];
    if constexpr (NU == 1) {
      dec8<DT>(vr[i][0], v);
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        v[4 * u] = __uint_as_float(vr[i][u].x); v[4 * u + 1] = __uint_as_float(vr[i][u].y);
        v[4 * u + 2] = __uint_as_float(vr[i][u].z); v[4 * u + 3] = __uint_as_float(vr[i][u].w);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = fmaf(p, v[e], o[e]);
  }
  // the row groups' sums: the two of each 16-lane DPP row by a rotation by
  // 8, then l over the four DPP rows; o's four DPP-row partials go to LDS
  l += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(l), 0x128, 0xf, 0xf, false));
  l = rows4_sum(l);
#pragma unroll
  for (int e = 0; e < 8; ++e)
    o[e] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(o[e]), 0x128, 0xf, 0xf, false));
  if (lane == 0) {
    wml[wave][0] = mx;
    wml[wave][1] = l;
  }
  if ((lane & 15) < 8 && dim_ok) {
#pragma unroll
    for (int e = 0; e < 8; ++e) wo[wave][lane >> 4][c * 8 + e] = o[e];
  }
  __syncthreads();
  if (tid < hd) {
    float m = wml[0][0];
#pragma unroll
    for (int w = 1; w < kSplit / 64; ++w) m = fmaxf(m, wml[w][0]);
    float ot = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < kSplit / 64; ++w) {
      const float f = wml[w][1] > 0.f ? __expf(wml[w][0] - m) : 0.f;
      const float ow = (wo[w][0][tid] + wo[w][1][tid]) + (wo[w][2][tid] + wo[w][3][tid]);
      ot = fmaf(ow, f, ot);
      lt = fmaf(wml[w][1], f, lt);
    }
    part_o[(long(bh) * ns + s) * hd + tid] = ot;
    if (tid == 0) part_ml[long(bh) * ns + s] = make_float2(m, lt);
  }
}

// After the last step of a call: the pending greedy choices (best[b]) become
// the next input and the generated tokens, best is reset and the position and
// step index advance (what the next step's first kernel does otherwise).
__global__ void __launch_bounds__(64)
dec_finish_kernel(unsigned long long *__restrict__ best, int32_t *__restrict__ ids, int32_t *__restrict__ tokens,
                  int *__restrict__ state, int B, int cap) {
  const int b = threadIdx.x;
  const int p0 = state[0], st = state[1], pend = state[2];
  if (!pend) return;  // (the same for every thread)
  if (b < B) {
    const unsigned long long k = best[b];
    const int out = k ? int(0xffffffffu - uint32_t(k & 0xffffffffu)) : 0;
    ids[b] = out;
    if (st < cap) tokens[long(st) * B + b] = out;
    best[b] = 0;
  }
  __syncthreads();
  if (b == 0) {
    state[0] = p0 + 1;
    state[1] = st + 1;
    state[2] = 0;
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

hipError_t dec_embed(int dt, int32_t *ids, unsigned long long *best, int32_t *tokens, int *state, const void *tok,
                     const void *pos_tab, void *out, int B, int V, int D, int cap, int *err, hipStream_t st) {
  if (B < 1 || B > 16 || D % int(16 / dt_size(dt)) != 0) return hipErrorInvalidValue;
  switch (dt) {
  case F32: hipLaunchKernelGGL(dec_embed_kernel<F32>, dim3(1), dim3(256), 0, st, ids, best, tokens, state, (const float *)tok, (const float *)pos_tab, (float *)out, B, V, D, cap, err); break;
  case F16: hipLaunchKernelGGL(dec_embed_kernel<F16>, dim3(1), dim3(256), 0, st, ids, best, tokens, state, (const uint16_t *)tok, (const uint16_t *)pos_tab, (uint16_t *)out, B, V, D, cap, err); break;
  case BF16: hipLaunchKernelGGL(dec_embed_kernel<BF16>, dim3(1), dim3(256), 0, st, ids, best, tokens, state, (const uint16_t *)tok, (const uint16_t *)pos_tab, (uint16_t *)out, B, V, D, cap, err); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// kind: 0 LayerNorm + q/k/v into q and the caches, 1 + residual, 2 LayerNorm
// + GELU, 3 LayerNorm + greedy argmax (the head), 4 attention shares +
// residual (the out-projection)
hipError_t dec_linear(int dt, int kind, const DecLinear &p, hipStream_t st) {
  const size_t es = dt_size(dt);
  const int ce = int(16 / es);
  if (p.M < 1 || p.M > 16 || p.K % ce != 0 || size_t(p.M) * p.K * es > 65536 || !p.bias) return hipErrorInvalidValue;
  const int KC = p.K / ce;
  if (kind == 4 && (p.nsplit < 1 || p.nsplit > kMaxSplit || p.hd % 4 != 0 || p.K % 4 != 0)) return hipErrorInvalidValue;
  DecLinArgs a{p.x, p.w, p.bias, p.ln_w, p.ln_b, p.resid, p.part_o, p.part_ml, p.out, p.kc, p.vc, p.best, p.state,
               p.pending, p.M, p.N, p.K, p.E, p.H, p.hd, p.Lmax, p.nsplit, p.eps, p.gelu_c};
  // Launch shape: K up to 128 chunks per column on one wave's 16-lane row
  // (up to 8 chunks per lane), longer K split over the block's four waves (up to
  // 512 chunks); the vocabulary head (N >= 8192, short K) takes 4 columns per
  // row so each block amortises its LayerNorm stage over 64 columns.  The
  // out-projection, whose 16-column blocks would leave CUs idle (48 blocks
  // at d 768), also splits K over four waves: four times the blocks, each
  // streaming a quarter of the bytes (5.19 -> 4.72 us at d 768, B 4).  The
  // LayerNorm-input products do not: four waves per column group slowed
  // QKV and FFN up from 4.8 to 12.9 us when their input stage held 8 chunks
  // per lane for every row, and the step from 0.257 to 0.280 ms with it sized
  // to K (two chunks): four times the blocks each repeat the LayerNorm stage.
  if (KC > 512) return hipErrorInvalidValue;
  const bool narrow = kind == 4 && (p.N + 15) / 16 < 256;
  const int ws = (KC > 128 || narrow) ? 4 : 1, cpl = (kind == 3 && ws == 1 && p.N >= 8192) ? 4 : 1;
  const bool few = p.M <= 4;
  const int ncols = (4 / ws) * 4 * cpl;  // columns per block
  const dim3 grid(unsigned((p.N + ncols - 1) / ncols));
  const size_t lds = size_t(p.M) * p.K * es;
  // weight chunk slots per lane: the K-chunks a lane takes, ceil(KC / (16
  // ws)), rounded up to 2, 6 or 8 (every slot is loaded, clamped past K: the
  // out-projection at d 768, two chunks per lane, loaded eight)
  const int need = (KC + 16 * ws - 1) / (16 * ws), kch = need <= 2 ? 2 : need <= 6 ? 6 : 8;
#define MH_DLK(DTV, KCV, MB, CPL, WS)                                                                                        \
  switch (kind) {                                                                                                            \
  case 0: hipLaunchKernelGGL((dec_linear_kernel<DTV, KCV, MB, CPL, WS, IN_LN, OUT_QKV, ACT_NONE, false>), grid, dim3(256), lds, st, a); break;   \
  case 1: hipLaunchKernelGGL((dec_linear_kernel<DTV, KCV, MB, CPL, WS, IN_ROW, OUT_ROW, ACT_NONE, true>), grid, dim3(256), lds, st, a); break;   \
  case 2: hipLaunchKernelGGL((dec_linear_kernel<DTV, KCV, MB, CPL, WS, IN_LN, OUT_ROW, ACT_GELU, false>), grid, dim3(256), lds, st, a); break;   \
  case 3: hipLaunchKernelGGL((dec_linear_kernel<DTV, KCV, MB, CPL, WS, IN_LN, OUT_ARGMAX, ACT_NONE, false>), grid, dim3(256), lds, st, a); break; \
  case 4: hipLaunchKernelGGL((dec_linear_kernel<DTV, KCV, MB, CPL, WS, IN_ATTN, OUT_ROW, ACT_NONE, true>), grid, dim3(256), lds, st, a); break;  \
  default: return hipErrorInvalidValue;                                                                                      \
  }
#define MH_DLW(DTV, KCV, MB)                                                     \
  if (ws == 4) {                                                                 \
    MH_DLK(DTV, KCV, MB, 1, 4)                                                   \
  } else if (cpl == 4) {                                                         \
    if (kind != 3) return hipErrorInvalidValue;                                  \
    hipLaunchKernelGGL((dec_linear_kernel<DTV, KCV, MB, 4, 1, IN_LN, OUT_ARGMAX, ACT_NONE, false>), grid, dim3(256), lds, st, a); \
  } else {                                                                       \
    MH_DLK(DTV, KCV, MB, 1, 1)                                                   \
  }
#define MH_DLS(DTV, MB)         \
  if (kch == 2) {               \
    MH_DLW(DTV, 2, MB)          \
  } else if (kch == 6) {        \
    MH_DLW(DTV, 6, MB)          \
  } else {                      \
    MH_DLW(DTV, 8, MB)          \
  }
#define MH_DL(DTV)              \
  if (few) {                    \
    MH_DLS(DTV, 4)              \
  } else {                      \
    MH_DLS(DTV, 16)             \
  }
  switch (dt) {
  case F32: MH_DL(F32); break;
  case F16: MH_DL(F16); break;
  case BF16: MH_DL(BF16); break;
  default: return hipErrorInvalidValue;
  }
#undef MH_DL
#undef MH_DLS
#undef MH_DLW
#undef MH_DLK
  return hipGetLastError();
}

hipError_t dec_attention(int dt, const void *q, const void *kc, const void *vc, const int *state, float *part_o,
                         float2 *part_ml, int B, int H, int hd, int Lmax, int blocks, float scale, hipStream_t st) {
  const int ns = blocks;
  // (eight lanes of 8 dimensions per key row)
  if (hd > 64 || hd % 8 != 0 || ns < 1 || ns > kMaxSplit || ns > (Lmax + kSplit - 1) / kSplit) return hipErrorInvalidValue;
  const dim3 grid(ns, B * H);
  switch (dt) {
  case F32: hipLaunchKernelGGL(dec_attn_kernel<F32>, grid, dim3(kSplit), 0, st, (const float *)q, (const float *)kc, (const float *)vc, state, part_o, part_ml, H, hd, Lmax, scale); break;
  case F16: hipLaunchKernelGGL(dec_attn_kernel<F16>, grid, dim3(kSplit), 0, st, (const uint16_t *)q, (const uint16_t *)kc, (const uint16_t *)vc, state, part_o, part_ml, H, hd, Lmax, scale); break;
  case BF16: hipLaunchKernelGGL(dec_attn_kernel<BF16>, grid, dim3(kSplit), 0, st, (const uint16_t *)q, (const uint16_t *)kc, (const uint16_t *)vc, state, part_o, part_ml, H, hd, Lmax, scale); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t dec_finish(unsigned long long *best, int32_t *ids, int32_t *tokens, int *state, int B, int cap,
                      hipStream_t st) {
  if (B < 1 || B > 16) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dec_finish_kernel, dim3(1), dim3(64), 0, st, best, ids, tokens, state, B, cap);
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
