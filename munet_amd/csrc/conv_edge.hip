// The convolutions at a conv network's two ends, where the implicit GEMM's
// tiles would be mostly padding and a layout conversion would be a launch of
// its own (ops::conv2d, reference src/core/ops/conv2d.cpp:8-103, with
// nn::Conv2d's bias, src/nn/linear.hpp:39-64):
//
// * conv3x3_fewc: a 3x3, stride-1, pad-1 convolution of an NCHW image with
//   at most 3 channels (K = 9 C <= 32: one 16-bit MFMA K step, or two fp32
//   groups of four) straight into an NHWC activation, bias + activation
//   fused: the NCHW -> NHWC copy of the image and its zero channel padding
//   are never written.
// * conv1x1_nchw: a 1x1 convolution of an NHWC activation to at most 8
//   channels (the output head) written straight as NCHW: the head's NHWC
//   output and its conversion are never written.
//
// Both keep the reference's convolution rounding: the fp32 accumulator plus
// the bias, one rounding to the storage dtype, then the activation
// (src/core/ops/conv2d.cpp:51-72 through the fp16/bf16 conversion fallback).
#include <cstdlib>

#include "gemm_common.hpp"
#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {
namespace {

// One wave: G groups of 16 output pixels (consecutive in N, H, W order) x
// 16 NT output channels, NT MFMAs v_mfma_f32_16x16x32 per group with the
// weights as the A operand (16 channels x 32 K) and the im2col values as the
// B operand (32 K x 16 pixels), so lane l ends with channels
// 16 t + 4 (l / 16) .. + 3 of pixel l % 16: four consecutive NHWC channels,
// one 8-byte store.  K index k = c 9 + kh 3 + kw, OIHW order, so the packed
// weights are the OIHW rows zero-padded to 32.  Lane l gathers K values
// 8 (l / 16) .. + 7 of its pixel: 2-byte loads (the image is small and
// cached), zero outside the image and past 9 C.  The weight fragments and
// biases are loaded once per wave and every gather of the G groups is
// issued before the first product.
template <int DT, int NT, int G>
__global__ void __launch_bounds__(256) conv3x3_fewc_kernel(const uint16_t *__restrict__ x,
                                                            const uint16_t *__restrict__ w, int B, int C, int H, int W,
                                                            EpiArgs ep) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  uint4 wf[NT];
  uint2 bb[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    wf[t] = *reinterpret_cast<const uint4 *>(w + (16 * t + li) * 32 + 8 * lg);
    bb[t] = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(ep.bias) + 16 * t + 4 * lg);
  }
  // this lane's 8 taps: channel plane offset and (dy, dx), or none
  int coff[8], dy[8], dx[8];
  bool tap[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * lg + e, c = k / 9, r = k - 9 * c;
    tap[e] = k < 9 * C;
    coff[e] = c * H * W;
    dy[e] = r / 3 - 1;
    dx[e] = r - 3 * (r / 3) - 1;
  }
  const long P = long(B) * H * W, HW = long(H) * W;
  const long p0 = (long(blockIdx.x) * 4 + wave) * (16 * G) + li;
  uint16_t v[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const long p = p0 + 16 * g, pc = p < P ? p : P - 1;
    const int b = int(pc / HW), hw = int(pc - b * HW), y = hw / W, xw = hw - y * W;
    const uint16_t *img = x + long(b) * C * HW;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int yy = y + dy[e], xx = xw + dx[e];
      const bool in = tap[e] && unsigned(yy) < unsigned(H) && unsigned(xx) < unsigned(W);
      v[g][e] = in ? img[coff[e] + yy * W + xx] : uint16_t(0);
    }
  }
  uint16_t *out = static_cast<uint16_t *>(ep.out);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    uint4 bv;
    bv.x = uint32_t(v[g][0]) | (uint32_t(v[g][1]) << 16);
    bv.y = uint32_t(v[g][2]) | (uint32_t(v[g][3]) << 16);
    bv.z = uint32_t(v[g][4]) | (uint32_t(v[g][5]) << 16);
    bv.w = uint32_t(v[g][6]) | (uint32_t(v[g][7]) << 16);
    const long p = p0 + 16 * g;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      Mfma<DT>::step(acc, wf[t], bv);
      float o[4] = {acc[0], acc[1], acc[2], acc[3]};
      const uint2 pk = epi_fast_value<DT>(ep, o, bb[t], make_uint2(0, 0));
      if (p < P) *reinterpret_cast<uint2 *>(out + p * ep.ldc + 16 * t + 4 * lg) = pk;
    }
  }
}

// The fp32 form (v_mfma_f32_16x16x4f32): lane l holds, per 16-wide K group
// g of the 32 (9 C <= 32), the 4 values k = 16 g + 4 (l / 16) .. + 3 of its
// pixel, and the four MFMAs of a group take element j of every lane (K
// contracted in that permuted order); one wave per 16 pixels, the general
// fp32 epilogue (bias added to the accumulator, the activation).
template <int NT>
__global__ void __launch_bounds__(256) conv3x3_fewc_f32_kernel(const float *__restrict__ x,
                                                                const float *__restrict__ w, int B, int C, int H, int W,
                                                                EpiArgs ep) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, q = lane >> 4;
  uint4 wf[NT][2];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 2; ++g) wf[t][g] = *reinterpret_cast<const uint4 *>(w + (16 * t + li) * 32 + 16 * g + 4 * q);
  const long P = long(B) * H * W, HW = long(H) * W;
  const long p = (long(blockIdx.x) * 4 + wave) * 16 + li, pc = p < P ? p : P - 1;
  const int b = int(pc / HW), hw = int(pc - b * HW), y = hw / W, xw = hw - y * W;
  const float *img = x + long(b) * C * HW;
  uint4 xv[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = 16 * g + 4 * q + j, c = k / 9, r = k - 9 * c;
      const int yy = y + r / 3 - 1, xx = xw + (r - 3 * (r / 3)) - 1;
      const bool in = k < 9 * C && unsigned(yy) < unsigned(H) && unsigned(xx) < unsigned(W);
      v[j] = in ? img[c * HW + long(yy) * W + xx] : 0.f;
    }
    xv[g] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    Mfma<F32>::step(acc, wf[t][0], xv[0]);
    Mfma<F32>::step(acc, wf[t][1], xv[1]);
    float o[4] = {acc[0], acc[1], acc[2], acc[3]};
    if (p < P) epi_store4<F32>(ep, int(p), 16 * t + 4 * q, 16 * NT, o, 0);
  }
}

// Sum over groups of LPP consecutive lanes (4, 8 or 16; every lane of a
// group gets it): the quad swaps, then the half-row and row mirrors.  Each
// step adds two equal-order partial sums, so every lane holds the same bits.
template <int LPP> __device__ __forceinline__ float lane_group_sum(float v) {
  static_assert(LPP == 4 || LPP == 8 || LPP == 16, "lanes per group");
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));   // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));   // quad [2,3,0,1]
  if constexpr (LPP >= 8)
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false));  // row_half_mirror
  if constexpr (LPP >= 16)
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xf, 0xf, false));  // row_mirror
  return v;
}

// 1x1 to oC <= 8 channels, NHWC in, NCHW out.  A pixel's iC channels are
// LPP = iC / 8 consecutive lanes' 16-byte chunks, so every load instruction
// reads 1 KB of contiguous activations; each lane forms its chunk's partial
// dot products for the oC outputs, the pixel's lanes add them with DPP
// (lane_group_sum), and the pixel's lane s writes output channels s,
// s + LPP, ...  U pixel groups per wave are loaded before the first product.
template <int DT, int LPP, int U>
__global__ void __launch_bounds__(256) conv1x1_nchw_kernel(const uint16_t *__restrict__ x,
                                                            const uint16_t *__restrict__ w,
                                                            const uint16_t *__restrict__ bias, uint16_t *__restrict__ out,
                                                            long M, int HW, long ldx, int oC, int act) {
  typedef Store<DT> S;
  constexpr int PPW = 64 / LPP;  // pixels per wave per group
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPP, pix = lane / LPP;
  const int c0 = sub * 8;
  const long base = (long(blockIdx.x) * 4 + wave) * (PPW * U);
  uint4 q[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long m = min(base + u * PPW + pix, M - 1);
    q[u] = *reinterpret_cast<const uint4 *>(x + m * ldx + c0);
  }
  float wl[8][8], bl[8];
#pragma unroll
  for (int o = 0; o < 8; ++o) {
    const uint4 qw = o < oC ? *reinterpret_cast<const uint4 *>(w + long(o) * (LPP * 8) + c0) : make_uint4(0, 0, 0, 0);
    const uint32_t wd[4] = {qw.x, qw.y, qw.z, qw.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) wl[o][e] = S::dec(uint16_t(wd[e >> 1] >> (16 * (e & 1))));
    bl[o] = o < oC ? S::dec(bias[o]) : 0.f;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t wd[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
    float xv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[e] = S::dec(uint16_t(wd[e >> 1] >> (16 * (e & 1))));
    float acc[8];
#pragma unroll
    for (int o = 0; o < 8; ++o) {
      acc[o] = 0.f;
      if (o < oC) {  // uniform
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a = __fmaf_rn(xv[e], wl[o][e], a);
        acc[o] = lane_group_sum<LPP>(a);
      }
    }
    const long m = base + u * PPW + pix;
    if (m < M) {
      const long b = m / HW, hw = m - b * HW;
#pragma unroll
      for (int o = 0; o < 8; ++o)
        if (o % LPP == sub && o < oC) {  // lane sub writes channels sub, sub + LPP, ...
          float v = S::round(acc[o] + bl[o]);
          if (act == ACT_RELU) v = v > 0.f ? v : 0.f;
          out[(b * oC + o) * HW + hw] = S::enc(v);
        }
    }
  }
}

}  // namespace

// Pixel groups per wave: MUNET_HIP_FEWC_G (16-pixel groups of the 3x3
// kernel: 1, 2 or 4) and MUNET_HIP_HEAD_U (groups of 64 / LPP pixels of the
// 1x1 kernel: 1, 2, 4 or 8), read once.  Measured on the UNet's 8 x 3 x
// 128 x 128 image (MI355X, kernel trace): the 3x3 kernel 13.3 / 15.0 /
// 21.1 us with 1 / 2 / 4 groups, the 1x1 head 10.8 / 10.0 / 16.3 us with
// 2 / 4 / 8 (the NCHW -> NHWC copy and general kernel they replace: 30.5 us;
// the one-pixel-per-thread head and NHWC -> NCHW copy: 18.0 us).
int edge_groups(const char *var, int dflt, int maxv) {
  const char *e = std::getenv(var);
  int v = e ? std::atoi(e) : dflt;
  if (v < 1 || v > maxv || (v & (v - 1))) v = dflt;
  return v;
}

bool conv3x3_fewc_ok(int dt, int C, int k, int s, int p, int oC) {
  return (dt == F16 || dt == BF16 || dt == F32) && C >= 1 && 9 * C <= 32 && k == 3 && s == 1 && p == 1 &&
         (oC == 16 || oC == 32 || oC == 64 || oC == 128);
}

hipError_t conv3x3_fewc(int dt, const void *x, const void *w32, int B, int C, int H, int W, int oC, const EpiArgs &ep,
                        hipStream_t st) {
  if (!conv3x3_fewc_ok(dt, C, 3, 1, 1, oC) || ep.mode != EPI_ROWMAJOR || ep.resid || !ep.bias_first || !ep.bias ||
      ep.ldc % 4 || (uintptr_t)ep.out % 8 || (uintptr_t)ep.bias % 8 || ep.act == ACT_GELU)
    return hipErrorInvalidValue;
  const long P = long(B) * H * W;
  if (P <= 0) return hipSuccess;
  if (dt == F32) {
    const long blocks = (P + 63) / 64;
    if (blocks > 0x7fffffffL) return hipErrorInvalidValue;
    const float *xf = static_cast<const float *>(x), *wf = static_cast<const float *>(w32);
    switch (oC) {
    case 16: hipLaunchKernelGGL(conv3x3_fewc_f32_kernel<1>, dim3(unsigned(blocks)), dim3(256), 0, st, xf, wf, B, C, H, W, ep); break;
    case 32: hipLaunchKernelGGL(conv3x3_fewc_f32_kernel<2>, dim3(unsigned(blocks)), dim3(256), 0, st, xf, wf, B, C, H, W, ep); break;
    case 64: hipLaunchKernelGGL(conv3x3_fewc_f32_kernel<4>, dim3(unsigned(blocks)), dim3(256), 0, st, xf, wf, B, C, H, W, ep); break;
    default: hipLaunchKernelGGL(conv3x3_fewc_f32_kernel<8>, dim3(unsigned(blocks)), dim3(256), 0, st, xf, wf, B, C, H, W, ep); break;
    }
    return hipGetLastError();
  }
  static const int G = edge_groups("MUNET_HIP_FEWC_G", 1, 4);
  const long blocks = (P + 64 * G - 1) / (64 * G);
  if (blocks > 0x7fffffffL) return hipErrorInvalidValue;
  const uint16_t *xi = static_cast<const uint16_t *>(x), *wi = static_cast<const uint16_t *>(w32);
#define MH_FEWC_G(DTV, NT, GV) \
  hipLaunchKernelGGL((conv3x3_fewc_kernel<DTV, NT, GV>), dim3(unsigned(blocks)), dim3(256), 0, st, xi, wi, B, C, H, W, ep)
#define MH_FEWC(DTV, NT)                     \
  if (G == 1) MH_FEWC_G(DTV, NT, 1);         \
  else if (G == 2) MH_FEWC_G(DTV, NT, 2);    \
  else MH_FEWC_G(DTV, NT, 4)
#define MH_FEWC_DT(DTV)           \
  switch (oC) {                   \
  case 16: MH_FEWC(DTV, 1); break; \
  case 32: MH_FEWC(DTV, 2); break; \
  case 64: MH_FEWC(DTV, 4); break; \
  default: MH_FEWC(DTV, 8); break; \
  }
  if (dt == F16) {
    MH_FEWC_DT(F16)
  } else {
    MH_FEWC_DT(BF16)
  }
#undef MH_FEWC_DT
#undef MH_FEWC
#undef MH_FEWC_G
  return hipGetLastError();
}

bool conv1x1_nchw_ok(int dt, int iC, long ldx, int oC) {
  return (dt == F16 || dt == BF16) && (iC == 32 || iC == 64 || iC == 128) && ldx % 8 == 0 && oC >= 1 && oC <= 8;
}

hipError_t conv1x1_nchw(int dt, const void *x, const void *w, const void *bias, void *out, long M, int HW, int iC,
                        long ldx, int oC, int act, hipStream_t st) {
  if (!conv1x1_nchw_ok(dt, iC, ldx, oC) || (uintptr_t)x % 16 || HW <= 0) return hipErrorInvalidValue;
  if (M <= 0) return hipSuccess;
  static const int U = edge_groups("MUNET_HIP_HEAD_U", 4, 8);
  const int ppb = 4 * (64 / (iC / 8)) * U;  // pixels per block
  const long blocks = (M + ppb - 1) / ppb;
  if (blocks > 0x7fffffffL) return hipErrorInvalidValue;
  const uint16_t *xi = static_cast<const uint16_t *>(x), *wi = static_cast<const uint16_t *>(w),
                 *bi = static_cast<const uint16_t *>(bias);
  uint16_t *o = static_cast<uint16_t *>(out);
#define MH_1X1_U(DTV, LPP, UV) \
  hipLaunchKernelGGL((conv1x1_nchw_kernel<DTV, LPP, UV>), dim3(unsigned(blocks)), dim3(256), 0, st, xi, wi, bi, o, M, HW, ldx, oC, act)
#define MH_1X1(DTV, LPP)                      \
  if (U == 1) MH_1X1_U(DTV, LPP, 1);          \
  else if (U == 2) MH_1X1_U(DTV, LPP, 2);     \
  else if (U == 4) MH_1X1_U(DTV, LPP, 4);     \
  else MH_1X1_U(DTV, LPP, 8)
#define MH_1X1_DT(DTV)            \
  switch (iC) {                   \
  case 32: MH_1X1(DTV, 4); break;  \
  case 64: MH_1X1(DTV, 8); break;  \
  default: MH_1X1(DTV, 16); break; \
  }
  if (dt == F16) {
    MH_1X1_DT(F16)
  } else {
    MH_1X1_DT(BF16)
  }
#undef MH_1X1_DT
#undef MH_1X1
#undef MH_1X1_U
  return hipGetLastError();
}

}  // namespace mh
