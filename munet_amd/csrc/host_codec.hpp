// Host-side restatement of MuNet's scalar codecs (reference
// src/types.hpp:239-317), used to round host constants (GELU's 1.702, the
// attention scale, masked_fill values) into a dtype before they reach a
// kernel, the way the reference stores them in a [1] tensor of that dtype.
#pragma once

#include <cstdint>
#include <cstring>

namespace mh {

inline uint16_t host_f32_to_bf16(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  b += 0x7fffu + ((b >> 16) & 1u);
  return uint16_t(b >> 16);
}

inline float host_bf16_to_f32(uint16_t h) {
  uint32_t b = uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

// Round half away from zero on the magnitude (same bit algorithm as the
// device encoder in mh_common.hpp).
inline uint16_t host_f32_to_f16(float f) {
  uint32_t bits;
  std::memcpy(&bits, &f, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t raw_exp = (bits >> 23) & 0xffu;
  uint32_t man = bits & 0x7fffffu;
  const int e = int(raw_exp) - 112;
  if (raw_exp == 0xffu) return uint16_t(sign | (man ? 0x7e00u : 0x7c00u));
  if (e <= 0) {
    if (e < -10) return uint16_t(sign);
    man |= 0x800000u;
    const uint32_t sh = man >> uint32_t(1 - e);
    return uint16_t(sign | ((sh + 0x1000u) >> 13));
  }
  const uint32_t v = (uint32_t(e) << 10) + ((man + 0x1000u) >> 13);
  if (v >= 0x7c00u) return uint16_t(sign | 0x7c00u);
  return uint16_t(sign | v);
}

inline float host_f16_to_f32(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      int sh = 0;
      while ((m & 0x400u) == 0) { m <<= 1; ++sh; }
      bits = sign | (uint32_t(113 - sh) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (e == 0x1fu) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// Value of `v` after storing it in a tensor of dtype dt (0 f32, 1 f16, 2 bf16).
inline float host_round(int dt, float v) {
  if (dt == 1) return host_f16_to_f32(host_f32_to_f16(v));
  if (dt == 2) return host_bf16_to_f32(host_f32_to_bf16(v));
  return v;
}

}  // namespace mh
