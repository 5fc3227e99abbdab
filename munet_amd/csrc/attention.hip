// Fused multi-head attention core for gfx950.
//
// Computes what nn::MultiHeadAttention::forward_impl does between the q/k/v
// projections and out_proj (reference src/nn/attention.hpp:51-99), without the
// dense [B*H*T]^2 scores and mask the reference materialises:
//
//   q, k, v : [B*H, T, hd] (the permute(0,2,1,3).contiguous() layout)
//   scores  = q.matmul(k.transpose(0,1))   -- the op layer hands the raw
//             contiguous k storage to the backend, so the right operand is
//             k's buffer read as a row-major [hd, B*H*T] matrix
//             (src/core/ops/matmul.cpp:331-392 ignores view strides):
//             S[i][j] = sum_d Q[bh][i][d] * Kflat[d*N + bh*T + j], N = B*H*T
//   scores *= scale (a [1] tensor of the dtype), then the block-diagonal /
//             causal mask with masked_fill(-1e9) and softmax(-1): masked
//             entries are exactly zero after exp, so each (b,h) block is an
//             independent softmax over its T columns (future columns masked
//             when causal).
//   ctx     = probs.matmul(v), merged back to [B, T, H*hd].
//
// Fast path (bf16/fp16, hd = 64): one workgroup of 4 wave64s owns QB query
// rows of one (b,h) block; KV tiles of 64 columns are staged through LDS in
// the MFMA operand layouts (K transposed to [j][d], V transposed to [d][j]);
// S^T = K*Q^T and O^T = V^T*P^T on v_mfma_f32_16x16x32 so that every lane owns
// one query row: the online-softmax max/sum need only two cross-lane shuffles
// and P goes from the S accumulators into the PV operand without touching LDS.
// Scores are rounded like the reference (round(matmul) then round(*scale)).
//
// Generic path (any dtype / head size): one wave per query row, scores kept in
// LDS, float max / double sum / per-j float accumulation as the reference's
// fp32 CPU kernels do (src/backend/cpu_backend.hpp:334-374, 587-611).
#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {

namespace {

constexpr int HD = 64;
constexpr int KB = 64;  // kv columns per tile

template <int DT> struct AttnMfma;
template <> struct AttnMfma<BF16> {
  static __device__ __forceinline__ void mma(f32x4 &c, uint4 a, uint4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                0, 0);
  }
  static __device__ __forceinline__ uint16_t cvt(float v) { return f32_to_bf16(v); }
};
template <> struct AttnMfma<F16> {
  static __device__ __forceinline__ void mma(f32x4 &c, uint4 a, uint4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                               0);
  }
  // P feeds the MFMA only; plain hardware RNE conversion is used here.
  static __device__ __forceinline__ uint16_t cvt(float v) {
    return __builtin_bit_cast(uint16_t, _Float16(v));
  }
};

// LDS tiles: 64 rows x 8 chunks of 16 bytes, chunk c of row r stored at
// c ^ (r & 7).
__device__ __forceinline__ int swz(int r, int c) { return r * 8 + (c ^ (r & 7)); }

template <int DT, int RW>
__global__ void __launch_bounds__(256)
flash_attn_kernel(const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K, const uint16_t *__restrict__ V,
                  uint16_t *__restrict__ O, int B, int H, int T, int causal, float scale) {
  typedef Store<DT> S;
  constexpr int QB = 4 * 16 * RW;
  __shared__ uint4 kt_lds[KB * 8];  // [j][d]
  __shared__ uint4 vt_lds[HD * 8];  // [d][j]

  const int bh = blockIdx.y;
  const int q0 = blockIdx.x * QB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const long N = long(B) * H * T;
  const uint16_t *Qb = Q + long(bh) * T * HD;
  const uint16_t *Vb = V + long(bh) * T * HD;
  const int wrow0 = q0 + wave * 16 * RW;

  // Q fragments (MFMA B operand): lane holds Q[i][8*(ks*4+lg) .. +8]
  uint4 qf[RW][2];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int i = wrow0 + r * 16 + li;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qf[r][ks] = (i < T) ? *reinterpret_cast<const uint4 *>(Qb + long(i) * HD + (ks * 4 + lg) * 8)
                          : make_uint4(0, 0, 0, 0);
    }
  }

  f32x4 o[RW][4];
  float mrow[RW], lrow[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    mrow[r] = -1e30f;
    lrow[r] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) o[r][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  int kv_end = T;
  if (causal) kv_end = min(T, q0 + QB);
  const int ntiles = (kv_end + KB - 1) / KB;
  const bool vec_ok = (T % 8) == 0;

  for (int t = 0; t < ntiles; ++t) {
    const int j0 = t * KB;
    __syncthreads();  // previous tile fully consumed
    // K slab: row d of the [hd, N] view holds 64 consecutive j at d*N+bh*T+j0
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int id = tid + it * 256, d = id >> 3, c = id & 7;
      const int j = j0 + c * 8;
      uint16_t vals[8];
      const uint16_t *src = K + long(d) * N + long(bh) * T + j;
      if (vec_ok && j + 8 <= T) {
        uint4 v = *reinterpret_cast<const uint4 *>(src);
        __builtin_memcpy(vals, &v, 16);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) vals[e] = (j + e < T) ? src[e] : uint16_t(0);
      }
      uint16_t *kl = reinterpret_cast<uint16_t *>(kt_lds);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int jj = c * 8 + e;
        kl[swz(jj, d >> 3) * 8 + (d & 7)] = vals[e];
      }
    }
    // V tile: rows j of [T, hd]; transposed into [d][j]
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int id = tid + it * 256, jj = id >> 3, c = id & 7;
      const int j = j0 + jj;
      uint4 v = (j < T) ? *reinterpret_cast<const uint4 *>(Vb + long(j) * HD + c * 8) : make_uint4(0, 0, 0, 0);
      uint16_t vals[8];
      __builtin_memcpy(vals, &v, 16);
      uint16_t *vl = reinterpret_cast<uint16_t *>(vt_lds);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = c * 8 + e;
        vl[swz(d, jj >> 3) * 8 + (jj & 7)] = vals[e];
      }
    }
    __syncthreads();

    if (causal && j0 > wrow0 + 16 * RW - 1) continue;  // whole wave masked

    // ---- S^T = K * Q^T : lane holds S[i=li][j = jt*16 + 4*lg + e] ----
    f32x4 s[RW][4];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) s[r][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const uint4 kf = kt_lds[swz(jt * 16 + li, ks * 4 + lg)];
#pragma unroll
        for (int r = 0; r < RW; ++r) AttnMfma<DT>::mma(s[r][jt], kf, qf[r][ks]);
      }
    }

    // ---- scale, mask, online softmax ----
    uint4 pf[RW][2];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int i = wrow0 + r * 16 + li;
      float mx = -1e30f;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = j0 + jt * 16 + lg * 4 + e;
          float v = S::round(S::round(s[r][jt][e]) * scale);
          const bool masked = (j >= T) || (causal && j > i);
          v = masked ? -INFINITY : v;
          s[r][jt][e] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(mrow[r], mx);
      const float alpha = __expf(mrow[r] - mnew);
      mrow[r] = mnew;
      float sum = 0.f;
      uint16_t pb[4][4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = __expf(s[r][jt][e] - mnew);
          sum += p;
          pb[jt][e] = AttnMfma<DT>::cvt(p);
        }
      sum += __shfl_xor(sum, 16, 64);
      sum += __shfl_xor(sum, 32, 64);
      lrow[r] = lrow[r] * alpha + sum;
#pragma unroll
      for (int d = 0; d < 4; ++d) o[r][d] *= alpha;
      // k-slot order for the PV step kk: j = 32kk + 4lg + {0..3}, 32kk + 16 + 4lg + {0..3}
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        uint16_t tmp[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          tmp[e] = pb[2 * kk][e];
          tmp[4 + e] = pb[2 * kk + 1][e];
        }
        __builtin_memcpy(&pf[r][kk], tmp, 16);
      }
    }

    // ---- O^T += V^T * P^T : lane holds O[i=li][d = dt*16 + 4*lg + e] ----
    const uint16_t *vl = reinterpret_cast<const uint16_t *>(vt_lds);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int d = dt * 16 + li;
        const int ja = kk * 32 + lg * 4, jb = ja + 16;
        const uint2 lo = *reinterpret_cast<const uint2 *>(vl + swz(d, ja >> 3) * 8 + (ja & 7));
        const uint2 hi = *reinterpret_cast<const uint2 *>(vl + swz(d, jb >> 3) * 8 + (jb & 7));
        const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int r = 0; r < RW; ++r) AttnMfma<DT>::mma(o[r][dt], vf, pf[r][kk]);
      }
    }
  }

  // ---- normalise, round, store merged [B, T, H*hd] ----
  const int b = bh / H, h = bh - b * H;
  const long E = long(H) * HD;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int i = wrow0 + r * 16 + li;
    if (i >= T) continue;
    const float inv = 1.0f / lrow[r];
    uint16_t *dst = O + (long(b) * T + i) * E + long(h) * HD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      u16x4 w;
      w.x = S::enc(o[r][dt][0] * inv);
      w.y = S::enc(o[r][dt][1] * inv);
      w.z = S::enc(o[r][dt][2] * inv);
      w.w = S::enc(o[r][dt][3] * inv);
      *reinterpret_cast<u16x4 *>(dst + dt * 16 + lg * 4) = w;
    }
  }
}

// Generic attention: one wave per (query row, bh); scores in LDS.
template <int DT>
__global__ void __launch_bounds__(64)
attn_generic_kernel(const void *__restrict__ Qv, const void *__restrict__ Kv, const void *__restrict__ Vv,
                    void *__restrict__ Ov, int B, int H, int T, int hd, int causal, float scale) {
  typedef Store<DT> S;
  typedef typename S::T T_;
  extern __shared__ float srow[];  // [T]
  const T_ *Q = static_cast<const T_ *>(Qv);
  const T_ *K = static_cast<const T_ *>(Kv);
  const T_ *V = static_cast<const T_ *>(Vv);
  T_ *O = static_cast<T_ *>(Ov);
  const int i = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  const long N = long(B) * H * T;
  const long qrow = (long(bh) * T + i) * hd;
  const int jend = causal ? i + 1 : T;
  float mx = -INFINITY;
  for (int j = lane; j < jend; j += 64) {
    float acc = 0.f;
    for (int d = 0; d < hd; ++d) acc += S::dec(Q[qrow + d]) * S::dec(K[long(d) * N + long(bh) * T + j]);
    const float v = S::round(S::round(acc) * scale);
    srow[j] = v;
    mx = fmaxf(mx, v);
  }
  mx = wave_max(mx);
  double sum = 0.0;
  for (int j = lane; j < jend; j += 64) sum += exp(double(srow[j]) - double(mx));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  __syncthreads();
  for (int j = lane; j < jend; j += 64) srow[j] = S::round(float(exp(double(srow[j]) - double(mx)) / sum));
  __syncthreads();
  const int b = bh / H, h = bh - b * H;
  for (int d = lane; d < hd; d += 64) {
    float acc = 0.f;
    for (int j = 0; j < jend; ++j) acc += srow[j] * S::dec(V[(long(bh) * T + j) * hd + d]);
    O[(long(b) * T + i) * (long(H) * hd) + long(h) * hd + d] = S::enc(acc);
  }
}

}  // namespace

hipError_t attention(int dt, const void *q, const void *k, const void *v, void *ctx, int B, int H, int T, int hd,
                     int causal, float scale, int force_generic, hipStream_t st) {
  if (B <= 0 || H <= 0 || T <= 0) return hipSuccess;
  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0) &&
                       ((uintptr_t)ctx % 8 == 0);
  if (!force_generic && hd == HD && (dt == BF16 || dt == F16) && aligned) {
    const int bh = B * H;
    // 128-row blocks when that still fills the chip, else 64-row blocks
    const int rw = (long((T + 127) / 128) * bh >= 512) ? 2 : 1;
    const int qb = 64 * rw;
    dim3 grid((T + qb - 1) / qb, bh);
    const uint16_t *Q = (const uint16_t *)q, *K = (const uint16_t *)k, *V = (const uint16_t *)v;
    uint16_t *O = (uint16_t *)ctx;
    if (dt == BF16) {
      if (rw == 2) hipLaunchKernelGGL((flash_attn_kernel<BF16, 2>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, scale);
      else hipLaunchKernelGGL((flash_attn_kernel<BF16, 1>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, scale);
    } else {
      if (rw == 2) hipLaunchKernelGGL((flash_attn_kernel<F16, 2>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, scale);
      else hipLaunchKernelGGL((flash_attn_kernel<F16, 1>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, scale);
    }
    return hipGetLastError();
  }
  if (size_t(T) * 4 > 64 * 1024) return hipErrorInvalidValue;
  dim3 grid(T, B * H);
  const size_t lds = size_t(T) * 4;
  switch (dt) {
  case F32: hipLaunchKernelGGL(attn_generic_kernel<F32>, grid, dim3(64), lds, st, q, k, v, ctx, B, H, T, hd, causal, scale); break;
  case F16: hipLaunchKernelGGL(attn_generic_kernel<F16>, grid, dim3(64), lds, st, q, k, v, ctx, B, H, T, hd, causal, scale); break;
  case BF16: hipLaunchKernelGGL(attn_generic_kernel<BF16>, grid, dim3(64), lds, st, q, k, v, ctx, B, H, T, hd, causal, scale); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mh
