// Implicit-GEMM convolution on the register-staged pipelined kernel
// (gemm_pipe.hpp, CONV): the conv2d of the reference's op layer
// (src/core/ops/conv2d.cpp, CPU semantics src/backend/cpu_backend.hpp:768-796)
// as M = B*oH*oW output pixels x N = oC x K = kH*kW*iC on an NHWC activation
// with OHWI weights.  The epilogue is the general program: the bias added to
// the fp32 accumulator and one rounding (conv), then the activation.
#include <cstdlib>

#include "gemm_pipe.hpp"

namespace mh {

namespace {

// Block tile: 64x64 (four waves of 32x32, 100 VGPRs, so several workgroups
// per CU hide the im2col gathers).  Measured on MI355X over the UNet's 13
// convolution shapes (131072 x 64 .. 2048 x 512 output pixels x channels, K
// 576 .. 4608): fastest or within 2% of the fastest on all but the small
// grids; 128x64 is up to 40% slower on the deep levels, 128x128 up to 90%
// slower.  Where 64x64 leaves at most one tile per CU and K <= 2304 (the
// stride-2 convolutions of the deep levels), 32x64 (four waves of 16x32)
// doubles the workgroups: 2048 x 256 x 2304 18.3 -> 14.2 us, 8192 x 128 x
// 1152 12.8 -> 11.5 us; with K = 4608 it was 11% slower.
int conv_tile(int M, int N, int K) {
  const long t64 = long((M + 63) / 64) * ((N + 63) / 64);
  return t64 <= 256 && K <= 2304 ? 3 : 2;
}

template <int DT>
hipError_t run(const void *x, const void *w, const ConvArgs &cv, int oC, const EpiArgs &ep, hipStream_t st) {
  const int M = cv.B * cv.oH * cv.oW;
  int tile = conv_tile(M, oC, cv.kH * cv.kW * cv.iC);
  // tuning override, read per call: MUNET_HIP_CONV_TILE = 0 128x128, 1 128x64, 2 64x64, 3 32x64, 4 64x32
  if (const char *e = std::getenv("MUNET_HIP_CONV_TILE")) {
    const int t = std::atoi(e);
    if (t >= 0 && t <= 4) tile = t;
  }
  switch (tile) {
  case 0: launch_conv<DT, 128, 128, 2, 2>(x, w, cv, oC, ep, st); break;
  case 1: launch_conv<DT, 128, 64, 2, 2>(x, w, cv, oC, ep, st); break;
  case 3: launch_conv<DT, 32, 64, 2, 2>(x, w, cv, oC, ep, st); break;
  case 4: launch_conv<DT, 64, 32, 2, 2>(x, w, cv, oC, ep, st); break;
  default: launch_conv<DT, 64, 64, 2, 2>(x, w, cv, oC, ep, st); break;
  }
  return hipGetLastError();
}

}  // namespace

bool gemm_pipe_conv_ok(int dt, const void *x, const void *w, const ConvArgs &cv) {
  const long xbytes = long(cv.B) * cv.iH * cv.iW * cv.ldx * 2;
  return (dt == BF16 || dt == F16) && cv.B > 0 && cv.iC > 0 && cv.iC % 64 == 0 && cv.ldx % 8 == 0 &&
         cv.ldx >= cv.iC && cv.kH > 0 && cv.kW > 0 && cv.kH * cv.kW <= 32 && cv.s > 0 && cv.oH > 0 && cv.oW > 0 &&
         (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 && xbytes + 16 < 0x7fffffffL &&
         long(cv.B) * cv.oH * cv.oW < 0x7fffffffL && long(cv.kH) * cv.kW * cv.iC < 0x7fffffffL;
}

hipError_t gemm_pipe_conv(int dt, const void *x, const void *w, const ConvArgs &cv, int oC, const EpiArgs &ep,
                          hipStream_t st) {
  if (oC <= 0 || long(cv.B) * cv.oH * cv.oW <= 0) return hipSuccess;
  if (!gemm_pipe_conv_ok(dt, x, w, cv) || ep.stats_out || ep.ln_stats) return hipErrorInvalidValue;
  if (long(oC - 1) * cv.kH * cv.kW * cv.iC + long(cv.kH) * cv.kW * cv.iC > 0xffffffffL) return hipErrorInvalidValue;
  return dt == BF16 ? run<BF16>(x, w, cv, oC, ep, st) : run<F16>(x, w, cv, oC, ep, st);
}

}  // namespace mh
