// Direct-to-LDS pipelined kernel on a 256x192 block tile with eight waves in
// a 4x2 grid (64x96 wave tiles, two waves per SIMD), two stages: tile 16.
// Eight waves per CU keep the matrix cores fed where the four-wave 128-row
// tiles leave them idle, and 256x192 covers a 4096x3072 product in exactly
// 256 tiles, one per CU.  Tile 19, 128x288 (32x144 wave tiles, three
// stages: 159.7 KB of the 160 KB LDS, the third stage measured 3 us faster
// per launch in the decoder forward), does the same for the 4096x2304 q/k/v
// product; tile 17, 128x96 with four
// stages, for the N = 768 products.  Every epilogue program (fixed bf16 ones and the
// general one); accumulators in VGPRs (see build.py).
#include "gemm_pipe.hpp"

namespace mh {

namespace {

template <int DT, int EK>
hipError_t run(int tile, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
               long sb, long sc, const EpiArgs &ep, hipStream_t st) {
  switch (tile) {
  case 16: launch_dma<DT, 256, 192, 4, 2, 2, EK>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 17: launch_dma<DT, 128, 96, 4, 2, 4, EK>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 19: launch_dma<DT, 128, 288, 4, 2, 3, EK>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t gemm_pipe_wide(int dt, int kind, int tile, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb,
                          int batch, long sa, long sb, long sc, const EpiArgs &ep, hipStream_t st) {
#define MH_RUN(EK) return run<BF16, EK>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st)
  if (dt == F16) {
    // fp16: the general program and the fixed ones without a folded LayerNorm
    switch (kind) {
    case PK_GENERAL: return run<F16, PK_GENERAL>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
    case PK_PLAIN: return run<F16, PK_PLAIN>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
    case PK_BIAS: return run<F16, PK_BIAS>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
    case PK_BIAS_GELU: return run<F16, PK_BIAS_GELU>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
    case PK_BIAS_RESID: return run<F16, PK_BIAS_RESID>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
    case PK_BIAS_NT: return run<F16, PK_BIAS_NT>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
    default: return hipErrorInvalidValue;
    }
  }
  switch (kind) {
  case PK_GENERAL: MH_RUN(PK_GENERAL);
  case PK_PLAIN: MH_RUN(PK_PLAIN);
  case PK_BIAS: MH_RUN(PK_BIAS);
  case PK_BIAS_GELU: MH_RUN(PK_BIAS_GELU);
  case PK_BIAS_RESID: MH_RUN(PK_BIAS_RESID);
  case PK_LN_BIAS: MH_RUN(PK_LN_BIAS);
  case PK_LN_BIAS_GELU: MH_RUN(PK_LN_BIAS_GELU);
  case PK_BIAS_RESID_ST: MH_RUN(PK_BIAS_RESID_ST);
  case PK_BIAS_NT: MH_RUN(PK_BIAS_NT);
  default: return hipErrorInvalidValue;
  }
#undef MH_RUN
}

}  // namespace mh
