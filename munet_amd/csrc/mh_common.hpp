// Shared device-side definitions for the MI355X (gfx950) kernels of the
// MuNet HIP backend: storage dtypes, the reference's rounding codecs, vector
// types for MFMA operands and small launch helpers.
//
// Storage formats follow MuNet (src/types.hpp:16-30): float32, float16 and
// bfloat16 are stored as 4/2/2-byte values, int32 for indices.  Rounding to a
// 16-bit storage type uses the reference's own codecs so that every op
// boundary rounds exactly like MuNet's CPU backend:
//   * fp16: round half away from zero on the magnitude
//     (src/types.hpp:239-278 adds half an ulp to the truncated mantissa);
//   * bf16: round to nearest even on the raw bits, with no NaN special case
//     (src/types.hpp:311-317).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mh_kernels.hpp"

namespace mh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

// ---- codecs ----------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(uint32_t(h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t b = __float_as_uint(f);
  b += 0x7fffu + ((b >> 16) & 1u);
  return uint16_t(b >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return float(v);
}

// fp16 encode with the reference's rounding: truncate the 23-bit mantissa to
// 10 bits after adding 0x1000 (half of the dropped 13-bit field), carrying into
// the exponent; subnormal results shift the implicit-one mantissa first and
// round the same way; overflow saturates to infinity; NaN becomes 0x7e00.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  const uint32_t bits = __float_as_uint(f);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t raw_exp = (bits >> 23) & 0xffu;
  uint32_t man = bits & 0x7fffffu;
  int e = int(raw_exp) - 112;  // rebias 127 -> 15
  if (raw_exp == 0xffu) return uint16_t(sign | (man ? 0x7e00u : 0x7c00u));
  if (e <= 0) {
    if (e < -10) return uint16_t(sign);
    man |= 0x800000u;
    const uint32_t sh = man >> uint32_t(1 - e);
    return uint16_t(sign | ((sh + 0x1000u) >> 13));
  }
  // normal: the carry out of the mantissa bumps the exponent naturally
  const uint32_t v = (uint32_t(e) << 10) + ((man + 0x1000u) >> 13);
  if (v >= 0x7c00u) return uint16_t(sign | 0x7c00u);
  return uint16_t(sign | v);
}

// The reference's fp16 rounding of a float, as a float (f16_to_f32 of
// f32_to_f16), without branches:
//  * normal half range [2^-14, 65520): adding 0x1000 and clearing the low 13
//    bits of the float's bits is MuNet's half-ulp rounding of the mantissa to
//    10 bits, the carry raising the exponent (the sign bit rides along);
//  * half subnormals [2^-25, 2^-14): multiples of 2^-24, half away from zero:
//    trunc(|x| 2^24 + 0.5) 2^-24 (exact: the sum only rounds below 2^-25);
//    below 2^-25, zero;
//  * 65520 and above: infinity; NaN: the quiet NaN MuNet's 0x7e00 decodes to.
__device__ __forceinline__ float round_f16_ref(float x) { return f16_to_f32(f32_to_f16(x)); }
__device__ __forceinline__ float round_f16_exact(float x) {
  const uint32_t b = __float_as_uint(x), a = b & 0x7fffffffu, s = b & 0x80000000u;
  const uint32_t rn = (b + 0x1000u) & 0xffffe000u;
  const float z = __builtin_truncf(__builtin_fmaf(__uint_as_float(a), 16777216.0f, 0.5f)) * 5.9604644775390625e-8f;
  const uint32_t rs = (a < 0x33000000u ? 0u : __float_as_uint(z)) | s;
  const uint32_t ro = (a > 0x7f800000u ? 0x7fc00000u : 0x7f800000u) | s;
  return __uint_as_float(a < 0x38800000u ? rs : a >= 0x477ff000u ? ro : rn);
}
// Four values at once: the 2-op normal-range rounding, and the full
// branch-free rounding for all four only when some lane of the wave has a
// value outside the normal half range [2^-14, 65520) (rare in practice;
// zero takes the full rounding too).  The range test is one clamp and one
// compare per value: med3(|x|, 2^-14, the float below 65520) == |x|.
__device__ __forceinline__ void round4_f16(float v[4]) {
  uint64_t slow = 0;  // lanes of the wave with a value outside the range (scalar masks)
  float r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t b = __float_as_uint(v[e]);
    r[e] = __uint_as_float((b + 0x1000u) & 0xffffe000u);
    const float t = __builtin_fabsf(v[e]);
    slow |= __builtin_amdgcn_ballot_w64(__builtin_amdgcn_fmed3f(t, 6.103515625e-05f, __uint_as_float(0x477fefffu)) != t);
  }
  if (slow) {
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = round_f16_exact(v[e]);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = r[e];
}

template <int DT> struct Store;
template <> struct Store<F32> {
  typedef float T;
  static __device__ __forceinline__ float load(const float *p, size_t i) { return p[i]; }
  static __device__ __forceinline__ float enc(float v) { return v; }
  static __device__ __forceinline__ float round(float v) { return v; }
  static __device__ __forceinline__ float dec(float v) { return v; }
};
template <> struct Store<F16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const uint16_t *p, size_t i) { return f16_to_f32(p[i]); }
  static __device__ __forceinline__ uint16_t enc(float v) { return f32_to_f16(v); }
  static __device__ __forceinline__ float round(float v) { return round_f16_exact(v); }
  static __device__ __forceinline__ float dec(uint16_t v) { return f16_to_f32(v); }
};
template <> struct Store<BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const uint16_t *p, size_t i) { return bf16_to_f32(p[i]); }
  static __device__ __forceinline__ uint16_t enc(float v) { return f32_to_bf16(v); }
  static __device__ __forceinline__ float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
  static __device__ __forceinline__ float dec(uint16_t v) { return bf16_to_f32(v); }
};

// Four consecutive values (8-byte aligned for 16-bit types, 16-byte for fp32)
// decoded to / encoded from floats with the dtype's codec.
template <int DT>
__device__ __forceinline__ void ld4(const typename Store<DT>::T *p, float v[4]) {
  if constexpr (DT == F32) {
    const f32x4 x = *reinterpret_cast<const f32x4 *>(p);
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
  } else {
    const u16x4 x = *reinterpret_cast<const u16x4 *>(p);
    v[0] = Store<DT>::dec(x[0]); v[1] = Store<DT>::dec(x[1]); v[2] = Store<DT>::dec(x[2]); v[3] = Store<DT>::dec(x[3]);
  }
}
template <int DT>
__device__ __forceinline__ void st4(typename Store<DT>::T *p, const float v[4]) {
  if constexpr (DT == F32) {
    *reinterpret_cast<f32x4 *>(p) = f32x4{v[0], v[1], v[2], v[3]};
  } else {
    u16x4 x;
    x[0] = Store<DT>::enc(v[0]); x[1] = Store<DT>::enc(v[1]); x[2] = Store<DT>::enc(v[2]); x[3] = Store<DT>::enc(v[3]);
    *reinterpret_cast<u16x4 *>(p) = x;
  }
}

// Generic (runtime dtype) scalar access for the cold paths.
__device__ __forceinline__ float ld_any(const void *p, int dt, size_t i) {
  if (dt == F32) return static_cast<const float *>(p)[i];
  if (dt == F16) return f16_to_f32(static_cast<const uint16_t *>(p)[i]);
  if (dt == BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
  return float(static_cast<const int32_t *>(p)[i]);
}

__device__ __forceinline__ void st_any(void *p, int dt, size_t i, float v) {
  if (dt == F32) static_cast<float *>(p)[i] = v;
  else if (dt == F16) static_cast<uint16_t *>(p)[i] = f32_to_f16(v);
  else if (dt == BF16) static_cast<uint16_t *>(p)[i] = f32_to_bf16(v);
  else static_cast<int32_t *>(p)[i] = int32_t(v);
}

// Sigmoid in float: 1 / (1 + e^-x), as the reference's fp32 kernel writes it
// (src/backend/cpu_backend.hpp:509-531).
// 1 / (1 + exp(-x)) as the reference writes it (src/nn/activations.hpp:31-38),
// with the hardware exp2 and reciprocal (within 2 ulp of the correctly rounded
// float expression; every caller rounds the result to the storage dtype or
// compares at fp32 tolerance).
__device__ __forceinline__ float sigmoidf_ref(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Wavefront (64-lane) reductions via cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum over the 16 lanes of a DPP row (every lane of the row gets it):
// rotate by 8 and 4 within the row, then the two quad swaps.  Reads only
// lanes of the same row, so rows whose lanes have all exited do not matter.
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));  // row_ror:8
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));   // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));   // quad [1,0,3,2]
  return v;
}

// The four DPP rows' values read from lanes 0, 16, 32 and 48 (the row's
// value must already be in its lane 0, 16, 32 or 48); every lane gets the
// same result.  Every lane of the wave must be active.
__device__ __forceinline__ float rows4_sum(float v) {
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}
__device__ __forceinline__ float rows4_max(float v) {
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Whole-wave sum without LDS-pipe shuffles: DPP within each 16-lane row,
// then the four rows through scalar reads (every lane gets the same value).
// Every lane of the wave must be active.
__device__ __forceinline__ float wave_sum_dpp(float v) { return rows4_sum(row16_sum(v)); }

// v[l] + v[l ^ 16] and v[l] + v[l ^ 32] through gfx950's VALU lane swaps
// instead of __shfl_xor's permute through the LDS pipe: v_permlane16_swap of v
// with itself leaves v[l] and v[l ^ 16] in its two results at every lane
// (the odd 16-lane rows of one operand traded with the even rows of the
// other), v_permlane32_swap v[l] and v[l ^ 32] (the halves traded); the sum
// of the two is the shuffle sum, bit for bit.  Every lane must be active.
__device__ __forceinline__ float xor16_add(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_add(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// fmaxf(v[l], v[l ^ 16]) and fmaxf(v[l], v[l ^ 32]) the same way
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Eight 16-bit values of one 16-byte chunk decoded to / encoded from floats.
template <int DT> __device__ __forceinline__ void dec8(uint4 c, float v[8]) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = Store<DT>::dec(uint16_t(w[i] & 0xffffu));
    v[2 * i + 1] = Store<DT>::dec(uint16_t(w[i] >> 16));
  }
}
// fp16 encodes through round4_f16 (the reference's rounding, the 2-op form
// unless a value of the wave is outside the normal half range) and packs the
// representable results exactly: the bits of Store<F16>::enc per value.
template <int DT> __device__ __forceinline__ uint4 enc8(const float v[8]) {
  uint32_t w[4];
  if constexpr (DT == F16) {
    float a[4] = {v[0], v[1], v[2], v[3]}, b[4] = {v[4], v[5], v[6], v[7]};
    round4_f16(a);
    round4_f16(b);
    w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a[0], a[1]));
    w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a[2], a[3]));
    w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(b[0], b[1]));
    w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(b[2], b[3]));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = uint32_t(Store<DT>::enc(v[2 * i])) | (uint32_t(Store<DT>::enc(v[2 * i + 1])) << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

inline size_t dtype_size(int dt) { return dt_size(dt); }

}  // namespace mh
