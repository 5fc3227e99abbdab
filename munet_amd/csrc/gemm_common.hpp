// Pieces shared by the MFMA GEMM kernels (gemm.hip, gemm_dma.hip): MFMA
// operand traits, the reference-rounding epilogue and the LDS-staged tile
// store.
#pragma once

#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {
namespace {

template <int DT> struct Mfma;
template <> struct Mfma<BF16> {
  static constexpr int kElems = 8;  // elements per 16-byte chunk
  static __device__ __forceinline__ void step(f32x4 &acc, uint4 a, uint4 b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma<F16> {
  static constexpr int kElems = 8;
  static __device__ __forceinline__ void step(f32x4 &acc, uint4 a, uint4 b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma<F32> {
  static constexpr int kElems = 4;
  static __device__ __forceinline__ void step(f32x4 &acc, uint4 a, uint4 b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
  }
};

// bf16 fast path: v_cvt_pk_bf16_f32 rounds two floats to nearest-even, the
// same rounding as MuNet's bf16 codec (src/types.hpp:311-317) for every
// non-NaN input.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
__device__ __forceinline__ float lo_bf16(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }
// round a float through bf16 with one instruction: packing (0, x) leaves
// bf16(x) in the high half and zero in the low half, i.e. round(x) as a float
__device__ __forceinline__ float round1_bf16(float x) { return __uint_as_float(pack_bf16x2(0.f, x)); }
// round 4 floats through bf16 in place
__device__ __forceinline__ void round4_inplace_bf16(float v[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = round1_bf16(v[i]);
}
// 4 floats -> packed bf16 (rounds; exact for values already rounded)
__device__ __forceinline__ uint2 pack4_bf16(const float v[4]) {
  return make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}

// fp16 counterparts: decode a packed pair, and pack two values that are
// already fp16-representable (the round-toward-zero conversion is then exact)
__device__ __forceinline__ float lo_f16(uint32_t p) { return f16_to_f32(uint16_t(p & 0xffffu)); }
__device__ __forceinline__ float hi_f16(uint32_t p) { return f16_to_f32(uint16_t(p >> 16)); }
__device__ __forceinline__ uint32_t pack_f16x2_exact(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// Destination of output element (m, n) for the epilogue modes.
// `off` is an element offset added to row-major outputs (the batch slice).
template <typename T>
__device__ __forceinline__ T *epi_dst(const EpiArgs &ep, int m, int n, long off) {
  if (ep.mode == EPI_HEADSPLIT) {
    const int which = n / ep.E, e = n - which * ep.E;
    const int h = e / ep.hd, dd = e - h * ep.hd;
    const int b = m / ep.T, t = m - b * ep.T;
    T *o = static_cast<T *>(which == 0 ? ep.outs[0] : which == 1 ? ep.outs[1] : ep.outs[2]);
    return o + ((long(b) * ep.H + h) * ep.T + t) * ep.hd + dd;
  }
  if (ep.mode == EPI_CONVT) {
    // column n = (kh*k + kw)*oC + oc of input pixel m = (b, ih, iw) lands on
    // output pixel (b, ih*k + kh, iw*k + kw) of an NHWC tensor (row stride ldc)
    const int oc = n % ep.convt_oc, ph = n / ep.convt_oc;
    const int kh = ph / ep.convt_k, kw = ph - kh * ep.convt_k;
    const int iw = m % ep.convt_iw, rest = m / ep.convt_iw;
    const int ih = rest % ep.convt_ih, b = rest / ep.convt_ih;
    const long opix = (long(b) * ep.convt_ih * ep.convt_k + ih * ep.convt_k + kh) * (long(ep.convt_iw) * ep.convt_k) +
                      iw * ep.convt_k + kw;
    return static_cast<T *>(ep.out) + opix * ep.ldc + oc;
  }
  return static_cast<T *>(ep.out) + off + long(m) * ep.ldc + n;
}

// Epilogue for C[m][n..n+3]: the reference's per-op rounding chain in
// registers -- round(matmul) -> round(+bias) -> activation -> round(+resid);
// GELU as x*round(sigmoid(round(x*c))) rounded (src/nn/activations.hpp:31-38);
// conv (bias_first) adds the bias to the fp32 accumulator and rounds once
// (src/core/ops/conv2d.cpp:51-72).
// Fast-path eligibility: bf16, a full 4-column group, row-major or head-split
// output, and 8-byte aligned bias / residual rows.
template <int DT> __device__ __forceinline__ bool epi_fast(const EpiArgs &ep, int n, int N) {
  return (DT == BF16 || DT == F16) && n + 4 <= N && ep.mode != EPI_CONVT && (!ep.resid || (ep.ldr & 3) == 0);
}

// The bf16 fast path's arithmetic: the rounded, packed 4 output values, with
// the bias and the residual already loaded (callers batch those loads).
// Intermediate results are rounded in place; the last one by the final pack.
__device__ __forceinline__ uint2 epi_fast_bf16_value(const EpiArgs &ep, float v[4], uint2 bias, uint2 resid) {
  if (ep.bias && ep.bias_first) {
    v[0] += lo_bf16(bias.x); v[1] += hi_bf16(bias.x); v[2] += lo_bf16(bias.y); v[3] += hi_bf16(bias.y);
    round4_inplace_bf16(v);
  } else {
    round4_inplace_bf16(v);
    if (ep.bias) {
      v[0] += lo_bf16(bias.x); v[1] += hi_bf16(bias.x); v[2] += lo_bf16(bias.y); v[3] += hi_bf16(bias.y);
      round4_inplace_bf16(v);
    }
  }
  if (ep.act == ACT_RELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = v[i] > 0.0f ? v[i] : 0.0f;  // exact on rounded values
  } else if (ep.act == ACT_GELU) {
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = v[i] * ep.gelu_c;
    round4_inplace_bf16(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = sigmoidf_ref(t[i]);
    round4_inplace_bf16(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] *= t[i];
    round4_inplace_bf16(v);
  }
  if (ep.resid) {
    v[0] = lo_bf16(resid.x) + v[0]; v[1] = hi_bf16(resid.x) + v[1];
    v[2] = lo_bf16(resid.y) + v[2]; v[3] = hi_bf16(resid.y) + v[3];
  }
  return pack4_bf16(v);
}

// The fp16 fast path: the same chain with the reference's fp16 rounding
// (round4_f16) after every op; the rounded values pack exactly.
__device__ __forceinline__ uint2 epi_fast_f16_value(const EpiArgs &ep, float v[4], uint2 bias, uint2 resid) {
  if (ep.bias && ep.bias_first) {
    v[0] += lo_f16(bias.x); v[1] += hi_f16(bias.x); v[2] += lo_f16(bias.y); v[3] += hi_f16(bias.y);
    round4_f16(v);
  } else {
    round4_f16(v);
    if (ep.bias) {
      v[0] += lo_f16(bias.x); v[1] += hi_f16(bias.x); v[2] += lo_f16(bias.y); v[3] += hi_f16(bias.y);
      round4_f16(v);
    }
  }
  if (ep.act == ACT_RELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = v[i] > 0.0f ? v[i] : 0.0f;  // exact on rounded values
  } else if (ep.act == ACT_GELU) {
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = v[i] * ep.gelu_c;
    round4_f16(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = sigmoidf_ref(t[i]);
    round4_f16(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] *= t[i];
    round4_f16(v);
  }
  if (ep.resid) {
    v[0] = lo_f16(resid.x) + v[0]; v[1] = hi_f16(resid.x) + v[1];
    v[2] = lo_f16(resid.y) + v[2]; v[3] = hi_f16(resid.y) + v[3];
    round4_f16(v);
  }
  return make_uint2(pack_f16x2_exact(v[0], v[1]), pack_f16x2_exact(v[2], v[3]));
}

template <int DT>
__device__ __forceinline__ uint2 epi_fast_value(const EpiArgs &ep, float v[4], uint2 bias, uint2 resid) {
  if constexpr (DT == F16) return epi_fast_f16_value(ep, v, bias, resid);
  else return epi_fast_bf16_value(ep, v, bias, resid);
}

// The same chain with the epilogue kind fixed at compile time (bias added
// after the matmul rounding, activation, residual): no runtime branches per
// fragment; every step but the last rounds in place (one instruction per
// value), the last step's rounding is the final pack.
template <bool BIAS, int ACT, bool RESID>
__device__ __forceinline__ uint2 epi_fast_bf16_fixed(float v[4], uint2 bias, uint2 resid, float gelu_c) {
  if constexpr (!BIAS && ACT == ACT_NONE && !RESID) return pack4_bf16(v);
  round4_inplace_bf16(v);
  if constexpr (BIAS) {
    v[0] += lo_bf16(bias.x); v[1] += hi_bf16(bias.x); v[2] += lo_bf16(bias.y); v[3] += hi_bf16(bias.y);
    if constexpr (ACT == ACT_NONE && !RESID) return pack4_bf16(v);
    round4_inplace_bf16(v);
  }
  if constexpr (ACT == ACT_RELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = v[i] > 0.0f ? v[i] : 0.0f;  // exact on rounded values
  } else if constexpr (ACT == ACT_GELU) {
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = v[i] * gelu_c;
    round4_inplace_bf16(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = sigmoidf_ref(t[i]);
    round4_inplace_bf16(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] *= t[i];
    if constexpr (!RESID) return pack4_bf16(v);
    round4_inplace_bf16(v);
  }
  if constexpr (RESID) {
    v[0] = lo_bf16(resid.x) + v[0]; v[1] = hi_bf16(resid.x) + v[1];
    v[2] = lo_bf16(resid.y) + v[2]; v[3] = hi_bf16(resid.y) + v[3];
  }
  return pack4_bf16(v);
}

// fp16: the same fixed chain with the reference's fp16 rounding (round4_f16)
// after every op, the last one included (the rounded values pack exactly);
// the bits of epi_fast_f16_value for the same chain.
template <bool BIAS, int ACT, bool RESID>
__device__ __forceinline__ uint2 epi_fast_f16_fixed(float v[4], uint2 bias, uint2 resid, float gelu_c) {
  round4_f16(v);
  if constexpr (BIAS) {
    v[0] += lo_f16(bias.x); v[1] += hi_f16(bias.x); v[2] += lo_f16(bias.y); v[3] += hi_f16(bias.y);
    round4_f16(v);
  }
  if constexpr (ACT == ACT_RELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = v[i] > 0.0f ? v[i] : 0.0f;  // exact on rounded values
  } else if constexpr (ACT == ACT_GELU) {
    float t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = v[i] * gelu_c;
    round4_f16(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] = sigmoidf_ref(t[i]);
    round4_f16(t);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] *= t[i];
    round4_f16(v);
  }
  if constexpr (RESID) {
    v[0] = lo_f16(resid.x) + v[0]; v[1] = hi_f16(resid.x) + v[1];
    v[2] = lo_f16(resid.y) + v[2]; v[3] = hi_f16(resid.y) + v[3];
    round4_f16(v);
  }
  return make_uint2(pack_f16x2_exact(v[0], v[1]), pack_f16x2_exact(v[2], v[3]));
}
template <int DT, bool BIAS, int ACT, bool RESID>
__device__ __forceinline__ uint2 epi_fast_fixed(float v[4], uint2 bias, uint2 resid, float gelu_c) {
  if constexpr (DT == F16) return epi_fast_f16_fixed<BIAS, ACT, RESID>(v, bias, resid, gelu_c);
  else return epi_fast_bf16_fixed<BIAS, ACT, RESID>(v, bias, resid, gelu_c);
}

// The 16-bit fast path for output columns n..n+3 of row m.
template <int DT>
__device__ __forceinline__ void epi_fast16(const EpiArgs &ep, int m, int n, float v[4], uint2 bias, uint2 resid,
                                           long off) {
  const uint2 pk = epi_fast_value<DT>(ep, v, bias, resid);
  uint16_t *dst = epi_dst<uint16_t>(ep, m, n, off);
  if (((uintptr_t)dst & 7) == 0) {
    *reinterpret_cast<uint2 *>(dst) = pk;
  } else {
    dst[0] = uint16_t(pk.x); dst[1] = uint16_t(pk.x >> 16); dst[2] = uint16_t(pk.y); dst[3] = uint16_t(pk.y >> 16);
  }
}

template <int DT>
__device__ __forceinline__ void epi_store4(const EpiArgs &ep, int m, int n, int N, float v[4], long off) {
  typedef Store<DT> S;
  typedef typename S::T T;
  const bool full = n + 4 <= N;
  if (epi_fast<DT>(ep, n, N)) {
    const uint2 b = ep.bias ? *reinterpret_cast<const uint2 *>(static_cast<const T *>(ep.bias) + n) : make_uint2(0, 0);
    const uint2 r = ep.resid ? *reinterpret_cast<const uint2 *>(static_cast<const T *>(ep.resid) + long(m) * ep.ldr + n)
                             : make_uint2(0, 0);
    epi_fast16<DT>(ep, m, n, v, b, r, off);
    return;
  }
  // generic path (fp32, fp16, tails, transposed-conv scatter)
  if (ep.bias && ep.bias_first) {
    const T *b = static_cast<const T *>(ep.bias);
    const int nb = ep.mode == EPI_CONVT ? ep.convt_oc : 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = S::round(v[i] + (n + i < N ? S::dec(b[(n + i) % nb]) : 0.0f));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = S::round(v[i]);
    if (ep.bias) {
      const T *b = static_cast<const T *>(ep.bias);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = S::round(v[i] + (n + i < N ? S::dec(b[n + i]) : 0.0f));
    }
  }
  if (ep.act == ACT_RELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = v[i] > 0.0f ? v[i] : 0.0f;
  } else if (ep.act == ACT_GELU) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float t1 = S::round(v[i] * ep.gelu_c);
      const float t2 = S::round(sigmoidf_ref(t1));
      v[i] = S::round(v[i] * t2);
    }
  }
  T *out = epi_dst<T>(ep, m, n, off);
  if (ep.resid) {
    const T *r = static_cast<const T *>(ep.resid) + long(m) * ep.ldr + n;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = S::round((n + i < N ? S::dec(r[i]) : 0.0f) + v[i]);
  }
  if (full && (((uintptr_t)out & (sizeof(T) * 4 - 1)) == 0)) {
    if (DT == F32) {
      *reinterpret_cast<float4 *>(out) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      u16x4 w;
      w.x = S::enc(v[0]); w.y = S::enc(v[1]); w.z = S::enc(v[2]); w.w = S::enc(v[3]);
      *reinterpret_cast<u16x4 *>(out) = w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n + i < N) out[i] = S::enc(v[i]);
  }
}

// Write a wave's accumulator tile (acc[i][j] = C[row0 + 16i + lane%16]
// [col0 + 16j + 4(lane/16) .. +3]) through the epilogue.  Each wave stages its
// accumulators through its own slice of the (idle) LDS in PASSES row bands,
// then streams each band back row by row: 4 consecutive columns per lane,
// consecutive lanes on consecutive columns, so global stores are contiguous
// row segments.  Fragment writes use compile-time accumulator indices only
// (keeps the accumulators in registers) and the epilogue body exists once.
template <int DT, int BM, int BN, int WTM, int WTN, int FM, int FN, int NW = 4>
__device__ __forceinline__ void store_tile(f32x4 (&acc)[FM][FN], float *lds, const EpiArgs &ep, int row0, int col0,
                                           int M, int N, int wave, int lane, long off) {
  constexpr int LDS_BYTES = 2 * (BM + BN) * 8 * 16;
  constexpr int RSTRIDE = WTN + 4;  // floats per staged row (+16 B pad)
  constexpr int PASSES = (NW * WTM * RSTRIDE * 4 <= LDS_BYTES) ? 1 : (NW * (WTM / 2) * RSTRIDE * 4 <= LDS_BYTES) ? 2 : 4;
  constexpr int FMP = FM / PASSES;
  static_assert(FM % PASSES == 0, "epilogue passes");
  float *stage = lds + wave * (FMP * 16) * RSTRIDE;
  const int lrow = lane & 15, lgrp = lane >> 4;
  constexpr int LPR = WTN / 4;   // lanes per staged row
  constexpr int RPI = 64 / LPR;  // rows per wave iteration
  // when LPR does not divide 64 the last lanes have no row of their own (they
  // would repeat rows of other lanes, which is wrong for in-place residuals)
  const int rl = lane < RPI * LPR ? lane / LPR : FMP * 16, cl = (lane % LPR) * 4;
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
#pragma unroll
    for (int i = 0; i < FMP; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        *reinterpret_cast<f32x4 *>(stage + (i * 16 + lrow) * RSTRIDE + j * 16 + lgrp * 4) = acc[p * FMP + i][j];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): own writes visible to own reads
    __builtin_amdgcn_wave_barrier();
    const int mbase = row0 + p * FMP * 16;
    const int n = col0 + cl;
    {
      for (int r = rl; r < FMP * 16; r += RPI) {
        const int m = mbase + r;
        if (m < M && n < N) {
          const f32x4 a = *reinterpret_cast<const f32x4 *>(stage + r * RSTRIDE + cl);
          float v[4] = {a[0], a[1], a[2], a[3]};
          epi_store4<DT>(ep, m, n, N, v, off);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace
}  // namespace mh
