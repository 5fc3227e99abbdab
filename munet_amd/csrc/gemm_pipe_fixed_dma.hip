// Fixed epilogue programs (PipeKind in gemm_pipe.hpp) of the direct-to-LDS
// pipelined kernel (bf16, and fp16 without a folded LayerNorm) on the tiles
// the automatic choice uses: 8 128x96 with 4 stages, 9 128x128 with 2
// stages.  Accumulators in VGPRs (see build.py).
#include "gemm_pipe.hpp"

namespace mh {

namespace {

template <int DT, int EK>
hipError_t run(int tile, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
               long sb, long sc, const EpiArgs &ep, hipStream_t st) {
  switch (tile) {
  case 8: launch_dma<DT, 128, 96, 2, 2, 4, EK>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 9: launch_dma<DT, 128, 128, 2, 2, 2, EK>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t gemm_pipe_fixed_dma(int dt, int kind, int tile, const void *A, const void *Bt, int M, int N, int K, long lda,
                               long ldb, int batch, long sa, long sb, long sc, const EpiArgs &ep, hipStream_t st) {
#define MH_RUN(EK) return run<BF16, EK>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st)
#define MH_RUN16(EK) return run<F16, EK>(tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st)
  if (dt == F16) {
    // fp16: the programs without a folded LayerNorm
    switch (kind) {
    case PK_PLAIN: MH_RUN16(PK_PLAIN);
    case PK_BIAS: MH_RUN16(PK_BIAS);
    case PK_BIAS_GELU: MH_RUN16(PK_BIAS_GELU);
    case PK_BIAS_RESID: MH_RUN16(PK_BIAS_RESID);
    case PK_BIAS_NT: MH_RUN16(PK_BIAS_NT);
    default: return hipErrorInvalidValue;
    }
  }
  switch (kind) {
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
#undef MH_RUN16
#undef MH_RUN
}

}  // namespace mh
