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
// Three kernels, chosen per call:
//  * flash_attn_tr_kernel (bf16/fp16, hd = 64, T % 8 == 0, power-of-two
//    scale -- the scale is round(1/sqrt(64)) = 0.125 for every hd = 64 call):
//    K and V tiles are copied to LDS in their natural layouts and the MFMA
//    operands are read back transposed with ds_read_b64_tr_b16;
//  * flash_attn_kernel (bf16/fp16, hd = 64, any T): transposes K and V while
//    writing them to LDS, and applies both score roundings;
//  * attn_generic_kernel (below).
// Both flash kernels compute S^T = K*Q^T and O^T = V^T*P^T on
// v_mfma_f32_16x16x32 so that every lane owns one query row: P goes from the
// S accumulators into the PV operand without touching LDS.  Scores are
// rounded like the reference (round(matmul), then round(*scale)).
//
// Generic path (any dtype / head size): one wave per query row, scores kept in
// LDS, float max / double sum / per-j float accumulation as the reference's
// fp32 CPU kernels do (src/backend/cpu_backend.hpp:334-374, 587-611).
#include <cmath>
#include <cstdlib>
#include <string>

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
  // two floats -> packed bf16 (hardware round-to-nearest-even)
  static __device__ __forceinline__ uint32_t cvt2(float a, float b) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, b2));
  }
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
  // two floats -> packed fp16 in one v_cvt_pk_f16_f32 (the same RNE as cvt)
  static __device__ __forceinline__ uint32_t cvt2(float a, float b) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, h2));
  }
};

// Round 4 floats through the storage dtype (MuNet's codecs; bf16 via the
// packed hardware RNE conversion, identical for non-NaN values).
template <int DT> __device__ __forceinline__ void round4(float v[4]);
template <> __device__ __forceinline__ void round4<BF16>(float v[4]) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  const uint32_t p0 = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{v[0], v[1]}, b2));
  const uint32_t p1 = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{v[2], v[3]}, b2));
  v[0] = __uint_as_float(p0 << 16); v[1] = __uint_as_float(p0 & 0xffff0000u);
  v[2] = __uint_as_float(p1 << 16); v[3] = __uint_as_float(p1 & 0xffff0000u);
}
// (MuNet's half-away codec: the 2-op normal-range form, the exact form only
// when some lane of the wave needs it; the same bits as Store<F16>::round)
template <> __device__ __forceinline__ void round4<F16>(float v[4]) { round4_f16(v); }

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

// ---------------------------------------------------------------------------
// Main path (bf16/fp16, hd = 64, T % 8 == 0, power-of-two scale).
//
// K and V tiles are staged in their natural layouts with 16-byte copies:
//   K tile [d][j] : 64 rows of the [64, B*H*T] slab view, 64 columns each
//   V tile [j][d] : 64 consecutive rows of the (b,h) block
// and the MFMA operands, which need 8 consecutive d (for K) or j (for V) per
// lane, are read with ds_read_b64_tr_b16.  Within each group of 16 lanes that
// instruction returns to lane i, element e, the value (i & 3) of the 8 bytes
// addressed by lane (i >> 2) + 4e, so a lane whose address names row
// R + 4h + (s >> 2), columns 4(s & 3).. of a row-major tile hands every lane i
// four consecutive rows of column i.
// Rows are 128 bytes; chunk c of row r is stored at chunk c ^ 2((r & 3) ^
// ((r >> SH) & 1)) (SH = 3 for K, 2 for V): the four rows one 16-lane group
// reads and the rows of the neighbouring group land on disjoint banks.
//
// Scores: the reference rounds q.k to the dtype and multiplies by the [1]
// scale tensor (rounded again); with a power-of-two scale that product is
// exact, so s = round(q.k) and the softmax runs in the log2 domain
// u = s * scale * log2(e).  The running max is only raised when it grows by
// more than 2^8 (p stays <= 256, exact enough for bf16 P and fp32 sums); row
// sums stay lane-partial until the end.
typedef short v4s __attribute__((ext_vector_type(4)));

template <int SH> __device__ __forceinline__ int tswz(int r, int c) {
  return r * 8 + (c ^ (2 * ((r & 3) ^ ((r >> SH) & 1))));
}

__device__ __forceinline__ uint2 lds_tr(const uint8_t *p) {
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)(p));
  return __builtin_bit_cast(uint2, r);
}

template <int V> struct BufIdx { static constexpr int value = V; };

template <int DT> __device__ __forceinline__ void round_scores(float v[4]) {
  if (DT == BF16) {
    round4<BF16>(v);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = Store<F16>::round(v[e]);
  }
}

// TXT (textbook keys): K is head-split like V, key j of block bh at row
// bh*T + j; its tile is staged in natural [j][d] layout (the swz pattern) and
// the MFMA's K operand is read straight, without the transposing read.
template <int DT, int RW, bool TXT>
__global__ void __launch_bounds__(256)
flash_attn_tr_kernel(const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K, const uint16_t *__restrict__ V,
                     uint16_t *__restrict__ O, int B, int H, int T, int causal, float c2) {
  constexpr int QB = 4 * 16 * RW;
  constexpr float kRaise = 8.0f;  // log2 of the largest unnormalised p
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][KB * HD * 2];  // [buf][K|V][tile]

  const int BH = B * H, nq = (T + QB - 1) / QB;
  const int lvl = blockIdx.x / BH, bh = blockIdx.x - lvl * BH;
  const int q0 = (causal ? nq - 1 - lvl : lvl) * QB;  // causal: longest rows first
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const long N = long(BH) * T;
  // column offset into the [64, N] slab, or the block's first key row (TXT)
  const uint16_t *Kb = TXT ? K + long(bh) * T * HD : K + long(bh) * T;
  const uint16_t *Vb = V + long(bh) * T * HD;
  const int wrow0 = q0 + wave * 16 * RW;

  // rows past T (ragged last block) read row T-1; their results are not stored
  uint4 qf[RW][2];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int i = min(wrow0 + r * 16 + li, T - 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      qf[r][ks] = *reinterpret_cast<const uint4 *>(Q + (long(bh) * T + i) * HD + ks * 32 + lg * 8);
  }
  // o: lane holds O[i = li][d = dt*16 + 4*lg + e]; osum: the row sum of the
  // (rounded) P fed to the MFMA, from a ones operand; mrow: running max (log2 units)
  f32x4 o[RW][4], osum[RW];
  float mrow[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    mrow[r] = -1e30f;
    osum[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 4; ++d) o[r][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t one2 = DT == BF16 ? 0x3F803F80u : 0x3C003C00u;
  const uint4 ones = make_uint4(one2, one2, one2, one2);

  // staging: rows r0 and r0 + 32 of each tile, chunk c0
  const int r0 = tid >> 3, c0 = tid & 7;
  const int st_k0 = (TXT ? swz(r0, c0) : tswz<3>(r0, c0)) * 16, st_k1 = (TXT ? swz(r0 + 32, c0) : tswz<3>(r0 + 32, c0)) * 16;
  const int st_v0 = tswz<2>(r0, c0) * 16, st_v1 = tswz<2>(r0 + 32, c0) * 16;
  // transposed reads: this lane addresses row base + (s >> 2), 8 bytes at
  // column 4(s & 3) of a 16-column block; the row swizzle term is lane-fixed
  const int s16 = lane & 15, sr = s16 >> 2, sx = ((s16 & 3) >> 1) ^ (2 * (sr ^ (lg & 1))), sh = (s16 & 1) * 8;
  const int rd_k = (8 * lg + sr) * 128 + sh;  // + (32ks + 4h) rows, chunk (2jt ^ sx)
  const int rd_v = (4 * lg + sr) * 128 + sh;  // + (32kk + 16h) rows, chunk (2dt ^ sx)

  const int kv_end = causal ? min(T, q0 + QB) : T;
  const int ntiles = (kv_end + KB - 1) / KB;
  // loop-carried load pointers (advanced one tile per gload) keep the address
  // registers live, so they are never recycled while a prefetch is in flight
  const long kld = TXT ? HD : N;  // elements between the rows of a K tile
  const uint16_t *kp0 = Kb + long(r0) * kld + c0 * 8, *kp1 = Kb + long(r0 + 32) * kld + c0 * 8;
  const uint16_t *vp0 = Vb + long(r0) * HD + c0 * 8, *vp1 = Vb + long(r0 + 32) * HD + c0 * 8;
  uint4 kr[2], vr[2];
  auto gload = [&](int j0) {
    if (j0 + KB <= T) {  // whole tile in range (wave-uniform)
      kr[0] = *reinterpret_cast<const uint4 *>(kp0);
      kr[1] = *reinterpret_cast<const uint4 *>(kp1);
      vr[0] = *reinterpret_cast<const uint4 *>(vp0);
      vr[1] = *reinterpret_cast<const uint4 *>(vp1);
    } else if (TXT) {  // ragged last tile: zero the rows past T
      kr[0] = (j0 + r0 < T) ? *reinterpret_cast<const uint4 *>(kp0) : make_uint4(0, 0, 0, 0);
      kr[1] = (j0 + r0 + 32 < T) ? *reinterpret_cast<const uint4 *>(kp1) : make_uint4(0, 0, 0, 0);
      vr[0] = (j0 + r0 < T) ? *reinterpret_cast<const uint4 *>(vp0) : make_uint4(0, 0, 0, 0);
      vr[1] = (j0 + r0 + 32 < T) ? *reinterpret_cast<const uint4 *>(vp1) : make_uint4(0, 0, 0, 0);
    } else {  // ragged last tile: zero what lies past T
      const bool kin = j0 + c0 * 8 < T;
      kr[0] = kin ? *reinterpret_cast<const uint4 *>(kp0) : make_uint4(0, 0, 0, 0);
      kr[1] = kin ? *reinterpret_cast<const uint4 *>(kp1) : make_uint4(0, 0, 0, 0);
      vr[0] = (j0 + r0 < T) ? *reinterpret_cast<const uint4 *>(vp0) : make_uint4(0, 0, 0, 0);
      vr[1] = (j0 + r0 + 32 < T) ? *reinterpret_cast<const uint4 *>(vp1) : make_uint4(0, 0, 0, 0);
    }
    kp0 += TXT ? KB * HD : KB;
    kp1 += TXT ? KB * HD : KB;
    vp0 += KB * HD;
    vp1 += KB * HD;
  };
  auto sstore = [&](int buf) {
    *reinterpret_cast<uint4 *>(&lds[buf][0][st_k0]) = kr[0];
    *reinterpret_cast<uint4 *>(&lds[buf][0][st_k1]) = kr[1];
    *reinterpret_cast<uint4 *>(&lds[buf][1][st_v0]) = vr[0];
    *reinterpret_cast<uint4 *>(&lds[buf][1][st_v1]) = vr[1];
  };
  if (ntiles > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();
  // The Q fragments arrived with the first tile (in-order completion).  Re-
  // defining them through an empty asm tells the wait-count insertion they
  // are settled, so the MFMAs of every tile do not wait for the prefetch.
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      asm volatile("" : "+v"(qf[r][ks].x), "+v"(qf[r][ks].y), "+v"(qf[r][ks].z), "+v"(qf[r][ks].w)::"memory");

  // one K/V tile; the LDS buffer index is a compile-time constant (the loop
  // below runs two tiles per trip) so the fragment addresses fold into
  // instruction offsets instead of being recomputed every tile
  auto tile = [&](int t, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int j0 = t * KB;
    if (t + 1 < ntiles) gload(j0 + KB);

    if (!(causal && j0 > wrow0 + 16 * RW - 1)) {  // skip tiles wholly above the diagonal
      const uint8_t *kt = lds[buf][0], *vt = lds[buf][1];
      // ---- S^T = K * Q^T : lane holds S[i = li][j = jt*16 + 4*lg + e] ----
      uint4 kf[2][4];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
          if constexpr (TXT) {
            kf[ks][jt] = *reinterpret_cast<const uint4 *>(kt + swz(jt * 16 + li, ks * 4 + lg) * 16);
          } else {
            const uint8_t *p = kt + rd_k + ((2 * jt) ^ sx) * 16 + ks * 32 * 128;
            const uint2 lo = lds_tr(p), hi = lds_tr(p + 4 * 128);
            kf[ks][jt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
          }
        }
      f32x4 s[RW][4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          s[r][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
          AttnMfma<DT>::mma(s[r][jt], kf[0][jt], qf[r][0]);
          AttnMfma<DT>::mma(s[r][jt], kf[1][jt], qf[r][1]);
        }

      uint4 pf[RW][2];
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        float v[16];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
          float w[4] = {s[r][jt][0], s[r][jt][1], s[r][jt][2], s[r][jt][3]};
          round_scores<DT>(w);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[jt * 4 + e] = w[e];
        }
        if (j0 + KB > T || (causal && j0 + KB - 1 > wrow0 + r * 16)) {  // boundary tile (wave-uniform)
          // element (jt, e) is column j0 + 4lg + jt*16 + e: masked past T or above the diagonal
          int lim = T - 1 - j0 - 4 * lg;
          if (causal) lim = min(lim, wrow0 + r * 16 + li - j0 - 4 * lg);
#pragma unroll
          for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (jt * 16 + e > lim) v[jt * 4 + e] = -INFINITY;
        }
        float mx = v[0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mx = fmaxf(mx, v[e]);
        // raise the row max only when some lane's own max exceeds it by 2^kRaise
        if (__any(mx * c2 > mrow[r] + kRaise)) {
          mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
          mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
          const float mnew = fmaxf(mrow[r], mx * c2);
          const float alpha = __builtin_amdgcn_exp2f(mrow[r] - mnew);
          mrow[r] = mnew;
          osum[r] *= alpha;
#pragma unroll
          for (int d = 0; d < 4; ++d) o[r][d] *= alpha;
        }
        const float nm = -mrow[r];
        uint32_t pk[8];
#pragma unroll
        for (int e = 0; e < 16; e += 2)
          pk[e >> 1] = AttnMfma<DT>::cvt2(__builtin_amdgcn_exp2f(__builtin_fmaf(v[e], c2, nm)),
                                          __builtin_amdgcn_exp2f(__builtin_fmaf(v[e + 1], c2, nm)));
        // P^T operand for k-step kk: slots 0..3 <- j = 32kk + 4lg + e, slots 4..7 <- j = 32kk + 16 + 4lg + e
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) pf[r][kk] = make_uint4(pk[4 * kk], pk[4 * kk + 1], pk[4 * kk + 2], pk[4 * kk + 3]);
      }

      // ---- O^T += V^T * P^T : lane holds O[i = li][d = dt*16 + 4*lg + e] ----
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        uint4 vf[4];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const uint8_t *p = vt + rd_v + ((2 * dt) ^ sx) * 16 + kk * 32 * 128;
          const uint2 lo = lds_tr(p), hi = lds_tr(p + 16 * 128);
          vf[dt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          AttnMfma<DT>::mma(osum[r], ones, pf[r][kk]);
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) AttnMfma<DT>::mma(o[r][dt], vf[dt], pf[r][kk]);
        }
      }
    }
    if (t + 1 < ntiles) sstore(buf ^ 1);
    __syncthreads();
  };
  int t = 0;
  for (; t + 1 < ntiles; t += 2) {
    tile(t, BufIdx<0>{});
    tile(t + 1, BufIdx<1>{});
  }
  if (t < ntiles) tile(t, BufIdx<0>{});

  const int b = bh / H, h = bh - b * H;
  const long E = long(H) * HD;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int i = wrow0 + r * 16 + li;
    if (i >= T) continue;
    const float inv = 1.0f / osum[r][0];
    uint16_t *dst = O + (long(b) * T + i) * E + long(h) * HD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      u16x4 w;
      w.x = Store<DT>::enc(o[r][dt][0] * inv);
      w.y = Store<DT>::enc(o[r][dt][1] * inv);
      w.z = Store<DT>::enc(o[r][dt][2] * inv);
      w.w = Store<DT>::enc(o[r][dt][3] * inv);
      *reinterpret_cast<u16x4 *>(dst + dt * 16 + lg * 4) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// Software-pipelined main path (bf16/fp16, hd = 64, T % 64 == 0, power-of-two
// scale, MuNet's K reading): the same tiles, transposing reads, log2-domain
// softmax and lazy max raise as flash_attn_tr_kernel, with the work of one
// 64-key tile spread over two loop trips so that a wave always has matrix and
// vector work in flight together:
//   trip t:  P(t) = exp2(S(t) c2 - m)          (VALU)
//            S(t+1) = K(t+1) Q^T               (MFMA, beside the exponentials)
//            O += V(t) P(t)^T                  (MFMA)
//            round / mask / lane max of S(t+1) (VALU, beside the PV MFMAs)
// K/V tiles rotate through three LDS buffers (tile t + 2 is written while
// tiles t and t + 1 are read), so a trip needs one barrier.  Trips past the
// last tile read stale buffers and re-load the last tile; their results are
// never used.  The score rounding takes one instruction per value: packing
// (0, x) to bf16 leaves round(x) as a float in the high half.
//
// Work order: items (query block, bh) heaviest first (causal), and within
// every odd round of `snake` workgroups (one per CU) the order is reversed in
// groups of 8, so the workgroups that share a CU pair heavy query blocks with
// light ones while each XCD keeps the same heads.
template <int DT> __device__ __forceinline__ float round1(float x);
template <> __device__ __forceinline__ float round1<BF16>(float x) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  return __uint_as_float(__builtin_bit_cast(uint32_t, __builtin_convertvector(f2{0.f, x}, b2)));
}
template <> __device__ __forceinline__ float round1<F16>(float x) { return Store<F16>::round(x); }

template <int DT>
__global__ void __launch_bounds__(256, 3)
flash_attn_pipe_kernel(const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K, const uint16_t *__restrict__ V,
                       uint16_t *__restrict__ O, int B, int H, int T, int causal, float c2, int snake) {
  constexpr float kRaise = 8.0f;  // log2 of the largest unnormalised p
  __shared__ __attribute__((aligned(16))) uint8_t lds[3][2][KB * HD * 2];  // [buf][K|V][tile]

  const int BH = B * H, nq = T / KB, n = nq * BH;
  int p = blockIdx.x;
  if (snake > 0) {
    const int r = p / snake;
    if (r & 1) {
      const int base = r * snake, cnt = min(n - base, snake), c = p - base;
      if ((cnt & 7) == 0) p = base + (cnt / 8 - 1 - c / 8) * 8 + (c & 7);
    }
  }
  const int lvl = p / BH, bh = p - lvl * BH;
  const int q0 = (causal ? nq - 1 - lvl : lvl) * KB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const long N = long(BH) * T;
  const uint16_t *Kb = K + long(bh) * T;  // column offset into the [64, N] slab
  const uint16_t *Vb = V + long(bh) * T * HD;
  const int wrow0 = q0 + wave * 16;

  uint4 qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qf[ks] = *reinterpret_cast<const uint4 *>(Q + (long(bh) * T + wrow0 + li) * HD + ks * 32 + lg * 8);
  f32x4 o[4], osum = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrow = -1e30f;
#pragma unroll
  for (int d = 0; d < 4; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t one2 = DT == BF16 ? 0x3F803F80u : 0x3C003C00u;
  const uint4 ones = make_uint4(one2, one2, one2, one2);

  // staging: rows r0 and r0 + 32 of each tile, chunk c0
  const int r0 = tid >> 3, c0 = tid & 7;
  const int st_k0 = tswz<3>(r0, c0) * 16, st_k1 = tswz<3>(r0 + 32, c0) * 16;
  const int st_v0 = tswz<2>(r0, c0) * 16, st_v1 = tswz<2>(r0 + 32, c0) * 16;
  const int s16 = lane & 15, sr = s16 >> 2, sx = ((s16 & 3) >> 1) ^ (2 * (sr ^ (lg & 1))), sh = (s16 & 1) * 8;
  const int rd_k = (8 * lg + sr) * 128 + sh;
  const int rd_v = (4 * lg + sr) * 128 + sh;

  const int ntiles = causal ? q0 / KB + 1 : nq;
  const uint16_t *kp0 = Kb + long(r0) * N + c0 * 8, *kp1 = Kb + long(r0 + 32) * N + c0 * 8;
  const uint16_t *vp0 = Vb + long(r0) * HD + c0 * 8, *vp1 = Vb + long(r0 + 32) * HD + c0 * 8;
  // staging registers as native vectors (HIP's uint4 is a struct: arrays of
  // it were copied through private memory); tile indices past the last tile
  // re-read the last tile
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(1))) const v4u gv4u;
  v4u kr0, kr1, vr0, vr1;
  auto gload = [&](int tile) {
    const int tt = min(tile, ntiles - 1);
    kr0 = *(gv4u *)(kp0 + tt * KB);
    kr1 = *(gv4u *)(kp1 + tt * KB);
    vr0 = *(gv4u *)(vp0 + tt * (KB * HD));
    vr1 = *(gv4u *)(vp1 + tt * (KB * HD));
  };
  auto sstore = [&](int buf) {
    *reinterpret_cast<v4u *>(&lds[buf][0][st_k0]) = kr0;
    *reinterpret_cast<v4u *>(&lds[buf][0][st_k1]) = kr1;
    *reinterpret_cast<v4u *>(&lds[buf][1][st_v0]) = vr0;
    *reinterpret_cast<v4u *>(&lds[buf][1][st_v1]) = vr1;
  };
  // S^T = K Q^T: lane holds S[i = li][j = jt*16 + 4*lg + e]
  auto kread = [&](const uint8_t *kt, uint4 (&kf)[2][4]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const uint8_t *p8 = kt + rd_k + ((2 * jt) ^ sx) * 16 + ks * 32 * 128;
        const uint2 lo = lds_tr(p8), hi = lds_tr(p8 + 4 * 128);
        kf[ks][jt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
  };
  auto kmma = [&](const uint4 (&kf)[2][4], f32x4 (&s)[4]) {
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      s[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
      AttnMfma<DT>::mma(s[jt], kf[0][jt], qf[0]);
    }
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) AttnMfma<DT>::mma(s[jt], kf[1][jt], qf[1]);
  };
  auto lane_max = [&](const float (&v)[16]) -> float {
    float mx = fmaxf(fmaxf(v[0], v[1]), v[2]);
#pragma unroll
    for (int e = 3; e < 15; e += 2) mx = fmaxf(fmaxf(mx, v[e]), v[e + 1]);
    return fmaxf(mx, v[15]);
  };
  // round the scores and take this lane's max
  auto round_scores16 = [&](const f32x4 (&s)[4], float (&v)[16]) -> float {
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      if constexpr (DT == BF16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[jt * 4 + e] = round1<DT>(s[jt][e]);
      } else {
        float w[4] = {s[jt][0], s[jt][1], s[jt][2], s[jt][3]};
        round4<DT>(w);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[jt * 4 + e] = w[e];
      }
    }
    return lane_max(v);
  };
  // the diagonal tile (j0 = q0): key j0 + 16 jt + 4 lg + e is masked above
  // row wrow0 + li; the max is taken again
  auto mask_diag = [&](float (&v)[16]) -> float {
    const int lim = wave * 16 + li - 4 * lg;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (jt * 16 + e > lim) v[jt * 4 + e] = -INFINITY;
    return lane_max(v);
  };

  gload(0);
  sstore(0);
  gload(1);
  sstore(1);
  gload(2);  // tile 2 (or the last tile again) in the staging registers
  __syncthreads();
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    asm volatile("" : "+v"(qf[ks].x), "+v"(qf[ks].y), "+v"(qf[ks].z), "+v"(qf[ks].w)::"memory");
  float v[16];
  float mx;
  {
    uint4 kf[2][4];
    f32x4 s0[4];
    kread(lds[0][0], kf);
    kmma(kf, s0);
    mx = round_scores16(s0, v);
    if (causal && ntiles == 1) mx = mask_diag(v);
  }

  // trip t: tile t's scores in v (rounded, masked) with this lane's max mx;
  // tile t in buffer bc, tile t + 1 in bn, tile t + 2 goes to bf
  auto trip = [&](int t, auto bcc, auto bnc, auto bfc) {
    constexpr int bc = decltype(bcc)::value, bn = decltype(bnc)::value, bf = decltype(bfc)::value;
    // raise the row max only when some lane's own max exceeds it by 2^kRaise
    // (a wave-uniform branch: every lane runs the lane swaps)
    if (__any(mx * c2 > mrow + kRaise)) {
      mx = xor32_max(xor16_max(mx));
      const float mnew = fmaxf(mrow, mx * c2);
      const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
      mrow = mnew;
      osum *= alpha;
#pragma unroll
      for (int d = 0; d < 4; ++d) o[d] *= alpha;
    }
    const float nm = -mrow;
    // one block: fragment reads, the exponentials beside S(t+1), the PV
    // MFMAs beside the staging and the rounding of S(t+1)
    uint4 kf[2][4];
    kread(lds[bn][0], kf);
    const uint8_t *vt = lds[bc][1];
    uint4 vf[2][4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint8_t *p8 = vt + rd_v + ((2 * dt) ^ sx) * 16 + kk * 32 * 128;
        const uint2 lo = lds_tr(p8), hi = lds_tr(p8 + 16 * 128);
        vf[kk][dt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
    uint32_t pk[8];
#pragma unroll
    for (int e = 0; e < 16; e += 2)
      pk[e >> 1] = AttnMfma<DT>::cvt2(__builtin_amdgcn_exp2f(__builtin_fmaf(v[e], c2, nm)),
                                      __builtin_amdgcn_exp2f(__builtin_fmaf(v[e + 1], c2, nm)));
    f32x4 sn[4];
    kmma(kf, sn);
    // (keeps the S MFMAs in phase 1: without a use here the instruction
    // selection may move them after the barrier below)
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) asm volatile("" : "+v"(sn[jt]));
    // phase 1: the 16 K fragment reads; 8 VALU; 8 x (S MFMA, 4 VALU, 2 V
    // fragment reads): the V reads spread over the phase instead of queueing
    // behind the K reads
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
    __builtin_amdgcn_sched_group_barrier(0x402, 8, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x402, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint4 pf = make_uint4(pk[4 * kk], pk[4 * kk + 1], pk[4 * kk + 2], pk[4 * kk + 3]);
      AttnMfma<DT>::mma(osum, ones, pf);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) AttnMfma<DT>::mma(o[dt], vf[kk][dt], pf);
    }
    sstore(bf);
    gload(t + 3);
    mx = round_scores16(sn, v);
    // phase 2: 10 x (PV MFMA, 3 VALU, one staging store or load)
#pragma unroll
    for (int i = 0; i < 10; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x402, 3, 0);
      if (i < 4) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      else if (i < 8) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    if (causal && t + 2 == ntiles) mx = mask_diag(v);
    __syncthreads();
  };
  int t = 0;
  for (; t + 3 <= ntiles; t += 3) {
    trip(t, BufIdx<0>{}, BufIdx<1>{}, BufIdx<2>{});
    trip(t + 1, BufIdx<1>{}, BufIdx<2>{}, BufIdx<0>{});
    trip(t + 2, BufIdx<2>{}, BufIdx<0>{}, BufIdx<1>{});
  }
  if (t < ntiles) trip(t, BufIdx<0>{}, BufIdx<1>{}, BufIdx<2>{});
  if (t + 1 < ntiles) trip(t + 1, BufIdx<1>{}, BufIdx<2>{}, BufIdx<0>{});

  const int b = bh / H, h = bh - b * H;
  const long E = long(H) * HD;
  const int i = wrow0 + li;
  const float inv = 1.0f / osum[0];
  uint16_t *dst = O + (long(b) * T + i) * E + long(h) * HD;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    u16x4 w;
    w.x = Store<DT>::enc(o[dt][0] * inv);
    w.y = Store<DT>::enc(o[dt][1] * inv);
    w.z = Store<DT>::enc(o[dt][2] * inv);
    w.w = Store<DT>::enc(o[dt][3] * inv);
    *reinterpret_cast<u16x4 *>(dst + dt * 16 + lg * 4) = w;
  }
}

// Generic attention: one wave per (query row, bh); scores in LDS.
template <int DT>
__global__ void __launch_bounds__(64)
attn_generic_kernel(const void *__restrict__ Qv, const void *__restrict__ Kv, const void *__restrict__ Vv,
                    void *__restrict__ Ov, int B, int H, int T, int hd, int causal, float scale, int textbook) {
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
    const long kj = textbook ? (long(bh) * T + j) * hd : long(bh) * T + j, kd = textbook ? 1 : N;
    for (int d = 0; d < hd; ++d) acc += S::dec(Q[qrow + d]) * S::dec(K[kj + long(d) * kd]);
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

namespace {
bool pow2(float x) {
  int e;
  return x > 0.f && std::frexp(x, &e) == 0.5f;
}
int tr_rows_env() {
  // tuning override: 1 or 2 (16 or 32 query rows per wave)
  const char *e = std::getenv("MUNET_HIP_ATTN_RW");
  const int v = e ? std::atoi(e) : 0;
  return (v == 1 || v == 2) ? v : 0;
}
// tuning overrides, read per call (so tests can compare the kernels in one
// process): MUNET_HIP_ATTN_KERNEL=tr keeps the single-trip flash kernel;
// MUNET_HIP_ATTN_ORDER=0 keeps the plain heaviest-first order
bool pipe_kernel_env() {
  const char *e = std::getenv("MUNET_HIP_ATTN_KERNEL");
  return !(e && std::string(e) == "tr");
}
bool snake_order_env() {
  const char *e = std::getenv("MUNET_HIP_ATTN_ORDER");
  return !(e && std::string(e) == "0");
}
// compute units of the current device (one workgroup round of the snake order)
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
    cached[dev] = cus > 0 ? cus : -1;
  }
  return cached[dev] > 0 ? cached[dev] : 0;
}
}  // namespace

hipError_t attention(int dt, const void *q, const void *k, const void *v, void *ctx, int B, int H, int T, int hd,
                     int causal, float scale, int force_generic, hipStream_t st, int textbook) {
  if (B <= 0 || H <= 0 || T <= 0) return hipSuccess;
  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) && ((uintptr_t)v % 16 == 0) &&
                       ((uintptr_t)ctx % 8 == 0);
  if (textbook && !force_generic && hd == HD && (dt == BF16 || dt == F16) && aligned && pow2(scale)) {
    // textbook keys: rows of K like V, so any T (ragged tiles are row-masked)
    const int bh = B * H;
    const dim3 grid(unsigned(long((T + 63) / 64) * bh));
    const float c2 = scale * 1.4426950408889634f;
    const uint16_t *Q = (const uint16_t *)q, *K = (const uint16_t *)k, *V = (const uint16_t *)v;
    uint16_t *O = (uint16_t *)ctx;
    if (dt == BF16) hipLaunchKernelGGL((flash_attn_tr_kernel<BF16, 1, true>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, c2);
    else hipLaunchKernelGGL((flash_attn_tr_kernel<F16, 1, true>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, c2);
    return hipGetLastError();
  }
  const bool use_pipe = pipe_kernel_env();
  if (use_pipe && !textbook && !force_generic && hd == HD && (dt == BF16 || dt == F16) && aligned && T % KB == 0 &&
      pow2(scale)) {
    const long items = long(T / KB) * B * H;
    if (items > 0x7fffffffL) return hipErrorInvalidValue;
    const bool snake_ok = snake_order_env();
    const int cus = cu_count();
    const int snake = (snake_ok && causal && cus > 0 && items > cus) ? cus : 0;
    const float c2 = scale * 1.4426950408889634f;
    const uint16_t *Q = (const uint16_t *)q, *K = (const uint16_t *)k, *V = (const uint16_t *)v;
    uint16_t *O = (uint16_t *)ctx;
    if (dt == BF16)
      hipLaunchKernelGGL((flash_attn_pipe_kernel<BF16>), dim3(unsigned(items)), dim3(256), 0, st, Q, K, V, O, B, H, T, causal, c2, snake);
    else
      hipLaunchKernelGGL((flash_attn_pipe_kernel<F16>), dim3(unsigned(items)), dim3(256), 0, st, Q, K, V, O, B, H, T, causal, c2, snake);
    return hipGetLastError();
  }
  if (!textbook && !force_generic && hd == HD && (dt == BF16 || dt == F16) && aligned && T % 8 == 0 && pow2(scale)) {
    const int bh = B * H;
    static const int forced = tr_rows_env();
    // 16 query rows per wave: more resident waves hide the softmax latency
    // better than the operand reuse of 32 rows per wave (measured on MI355X)
    const int rw = forced ? forced : 1;
    const int qb = 64 * rw;
    const dim3 grid(unsigned(long((T + qb - 1) / qb) * bh));
    const float c2 = scale * 1.4426950408889634f;
    const uint16_t *Q = (const uint16_t *)q, *K = (const uint16_t *)k, *V = (const uint16_t *)v;
    uint16_t *O = (uint16_t *)ctx;
    if (dt == BF16) {
      if (rw == 2) hipLaunchKernelGGL((flash_attn_tr_kernel<BF16, 2, false>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, c2);
      else hipLaunchKernelGGL((flash_attn_tr_kernel<BF16, 1, false>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, c2);
    } else {
      if (rw == 2) hipLaunchKernelGGL((flash_attn_tr_kernel<F16, 2, false>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, c2);
      else hipLaunchKernelGGL((flash_attn_tr_kernel<F16, 1, false>), grid, dim3(256), 0, st, Q, K, V, O, B, H, T, causal, c2);
    }
    return hipGetLastError();
  }
  if (!textbook && !force_generic && hd == HD && (dt == BF16 || dt == F16) && aligned) {
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
  case F32: hipLaunchKernelGGL(attn_generic_kernel<F32>, grid, dim3(64), lds, st, q, k, v, ctx, B, H, T, hd, causal, scale, textbook); break;
  case F16: hipLaunchKernelGGL(attn_generic_kernel<F16>, grid, dim3(64), lds, st, q, k, v, ctx, B, H, T, hd, causal, scale, textbook); break;
  case BF16: hipLaunchKernelGGL(attn_generic_kernel<BF16>, grid, dim3(64), lds, st, q, k, v, ctx, B, H, T, hd, causal, scale, textbook); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mh
