// The direct-to-LDS pipelined kernel (gemm_pipe.hpp) on a 256x256 block tile
// for wide, shallow products such as the vocabulary head (4096 x 32000 x 768):
// four waves in a 2x2 grid, each owning a 128x128 wave tile, two 64 KB
// stages.  A 256x256 tile reads 2 * 256 * 64 * 2 bytes per 64-wide K step
// for 2 * 256 * 256 * 64 FLOPs (128 FLOP per byte, twice the 128x128
// tile's), so the per-CU feed from L2 is no longer the limit.  Each lane
// holds 256 accumulator registers, which live in AGPRs (this source is built
// without -amdgpu-mfma-vgpr-form) beside the fragment registers; one
// workgroup per CU.  Programs: plain, bias, bias with non-temporal stores.
#include "gemm_pipe.hpp"

namespace mh {

namespace {

template <int EK>
hipError_t run(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa, long sb,
               long sc, const EpiArgs &ep, hipStream_t st) {
  launch_dma<BF16, 256, 256, 2, 2, 2, EK>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  return hipGetLastError();
}

}  // namespace

hipError_t gemm_pipe_head(int kind, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                          long sa, long sb, long sc, const EpiArgs &ep, hipStream_t st) {
  switch (kind) {
  case PK_PLAIN: return run<PK_PLAIN>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  case PK_BIAS: return run<PK_BIAS>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  case PK_BIAS_NT: return run<PK_BIAS_NT>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  default: return hipErrorNotSupported;
  }
}

}  // namespace mh
