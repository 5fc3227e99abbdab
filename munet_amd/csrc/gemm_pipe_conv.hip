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

// Block tile and kernel per shape, measured on MI355X over the UNet's
// convolutions (kernel trace, fp16, B 8; profiles/unet_forward_kernel_stats.md
// has the sweeps):
//  * the 128x128 maps (M = 131072 output pixels): direct-to-LDS 256x64 with
//    eight waves and two stages (enc0.1 25.7 -> 21.8 us, dec0.0 39.0 -> 31.5,
//    dec0.1 28.4 -> 24.1 against the register-staged 64x64 four-wave tile);
//  * the 64x64 maps (M = 32768) and the 32x32 maps with N >= 256: direct-to-LDS
//    128x64 with eight waves and three stages (enc1.1 19.8 -> 17.4, dec2.0
//    32.4 -> 28.8, enc2.1 19.3 -> 17.3 against the four-wave 64x128 / 64x64
//    tiles), or 128x128 with eight waves and three stages for N >= 128 and
//    K > 1152 (dec1.0 28.4 -> 26.9): eight waves per workgroup share each
//    weight slab between twice the output pixels;
//  * the deeper maps, where a larger tile leaves CUs idle: direct-to-LDS with
//    four waves and four stages, 32x64 when 64x64 leaves fewer than 256 tiles,
//    or exactly 256 with K <= 2304 (down2 11.6, enc3.0 14.4, down1 10.9 us),
//    else 64x64 (enc3.1 23.0).
// Every tile gives the same bits (test_conv_pipelined_kernel_bits).
int conv_tile(int M, int N, int K) {
  const long t64 = long((M + 63) / 64) * ((N + 63) / 64);
  if (M >= 65536) return 10;
  if (M >= 16384) return N >= 128 && K > 1152 ? 11 : 9;
  if (M >= 8192 && N >= 256) return 9;
  return t64 < 256 || (t64 == 256 && K <= 2304) ? 6 : 5;
}

template <int DT>
hipError_t run(const void *x, const void *w, const ConvArgs &cv, int oC, const EpiArgs &ep, hipStream_t st) {
  const int M = cv.B * cv.oH * cv.oW;
  int tile = conv_tile(M, oC, cv.kH * cv.kW * cv.iC);
  // tuning override, read per call: MUNET_HIP_CONV_TILE = 0 128x128, 1 128x64, 2 64x64, 3 32x64, 4 64x32
  // (register-staged), 5 64x64 four stages, 6 32x64 four stages, 7 64x64 three stages, 8 64x128 three
  // stages (direct-to-LDS, four waves), 9 128x64 three stages, 10 256x64 two stages, 11 128x128 three
  // stages (direct-to-LDS, eight waves)
  if (const char *e = std::getenv("MUNET_HIP_CONV_TILE")) {
    const int t = std::atoi(e);
    if (t >= 0 && t <= 11) tile = t;
  }
  switch (tile) {
  case 9: launch_dma_conv<DT, 128, 64, 4, 2, 3>(x, w, cv, oC, ep, st); break;
  case 10: launch_dma_conv<DT, 256, 64, 4, 2, 2>(x, w, cv, oC, ep, st); break;
  case 11: launch_dma_conv<DT, 128, 128, 4, 2, 3>(x, w, cv, oC, ep, st); break;
  case 5: launch_dma_conv<DT, 64, 64, 2, 2, 4>(x, w, cv, oC, ep, st); break;
  case 6: launch_dma_conv<DT, 32, 64, 2, 2, 4>(x, w, cv, oC, ep, st); break;
  case 7: launch_dma_conv<DT, 64, 64, 2, 2, 3>(x, w, cv, oC, ep, st); break;
  case 8: launch_dma_conv<DT, 64, 128, 2, 2, 3>(x, w, cv, oC, ep, st); break;
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
