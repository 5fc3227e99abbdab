// Pipelined 16-bit MFMA GEMM kernels (gemm_pipe.hpp) with 256-row block
// tiles: four waves in a 2x2 grid, each owning a 128 x BN/2 wave tile, which
// reads (8 + BN/32) fragments from LDS per 8 * BN/32 MFMAs (a 64x64 wave tile
// 8 per 16).  Their 128-192 accumulator registers per lane live in AGPRs
// (this source is built without -amdgpu-mfma-vgpr-form), which leaves the
// VGPRs to the staging and fragment registers.  (A 256x256 tile spills even
// so, and is not instantiated.)
#include "gemm_pipe.hpp"

namespace mh {

namespace {

template <int DT>
hipError_t launch_big(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
                      long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st) {
  switch (tile) {
  case 1: launch<DT, 256, 192, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 2: launch<DT, 256, 128, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 10: launch_dma<DT, 256, 192, 2, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 11: launch_dma<DT, 256, 128, 2, 2, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t gemm_pipe_big(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                         long sa, long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st) {
  if (dt == BF16) return launch_big<BF16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile, st);
  if (dt == F16) return launch_big<F16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile, st);
  return hipErrorInvalidValue;
}

}  // namespace mh
