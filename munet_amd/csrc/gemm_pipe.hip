// Pipelined 16-bit MFMA GEMM (gemm_pipe.hpp), block tiles up to 128 rows with
// the accumulators in ordinary VGPRs (built with -amdgpu-mfma-vgpr-form, see
// build.py), and the tile dispatcher for the pipelined kernels.  256-row
// tiles are instantiated in gemm_pipe_big.hip.
#include "gemm_pipe.hpp"

namespace mh {

namespace {

template <int DT>
hipError_t launch_dt(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
                     long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st) {
  if (tile < 0) {
    // measured on MI355X (decoder shapes, K = 768 / 3072, M = 4096):
    //  * N tiling evenly by 96 with at most one tile per CU (N = 768: FFN down,
    //    attention out-projection): direct-to-LDS 128x96, 4 stages (one
    //    workgroup per CU, so deep stages hide the memory latency);
    //  * at least 8 tiles per CU at 128x128 (the LM head): direct-to-LDS
    //    128x128, 2 stages (two workgroups per CU);
    //  * otherwise register-staged: 128x128 when N tiles evenly by 128 and
    //    there are >= 2.5 tiles per CU (FFN up), 128x96 when N tiles evenly
    //    by 96 (QKV), else 128x128 / 128x64 / 64x64 by tile count.
    const bool dma = gemm_pipe_dma_ok(A, Bt, M, N, K, lda, ldb);
    const long t128 = long((M + 127) / 128) * ((N + 127) / 128) * batch;
    const long t96 = long((M + 127) / 128) * ((N + 95) / 96) * batch;
    const long t64 = long((M + 127) / 128) * ((N + 63) / 64) * batch;
    if (dma && N % 96 == 0 && t96 <= 256) tile = 8;
    else if (dma && N % 128 == 0 && t128 >= 2048) tile = 9;
    else if (N % 128 == 0 && t128 >= 640) tile = 0;
    else if (N % 96 == 0) tile = 3;
    else tile = (t128 >= 640 || (K >= 2048 && t128 >= 128)) ? 0 : (t64 >= 256 ? 1 : 2);
  }
  if (tile >= 7 && !gemm_pipe_dma_ok(A, Bt, M, N, K, lda, ldb)) tile = 0;
  if (tile >= 4 && tile <= 6) return gemm_pipe_big(DT, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile - 4, st);
  if (tile >= 13) return gemm_pipe_big(DT, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile - 4, st);
  switch (tile) {
  case 0: launch<DT, 128, 128, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 1: launch<DT, 128, 64, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 3: launch<DT, 128, 96, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 7: launch_dma<DT, 128, 128, 2, 2, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 8: launch_dma<DT, 128, 96, 2, 2, 4>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 9: launch_dma<DT, 128, 128, 2, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 10: launch_dma<DT, 128, 96, 2, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 11: launch_dma<DT, 128, 96, 2, 2, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 12: launch_dma<DT, 128, 64, 2, 2, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  default: launch<DT, 64, 64, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  }
  return hipGetLastError();
}

}  // namespace

bool gemm_pipe_ok(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, long sa, long sb) {
  // per-thread 32-bit element offsets: the last row's last slab must be
  // addressable from the slab base
  const bool fits = M > 0 && N > 0 && long(M - 1) * lda + K <= 0xffffffffL && long(N - 1) * ldb + K <= 0xffffffffL;
  return (dt == BF16 || dt == F16) && K > 0 && K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && sa % 8 == 0 &&
         sb % 8 == 0 && (uintptr_t)A % 16 == 0 && (uintptr_t)Bt % 16 == 0 && fits;
}

bool gemm_pipe_dma_ok(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb) {
  // K in whole 64-wide slabs; per-lane 32-bit byte offsets from the slab base
  return K % 64 == 0 && (long(M - 1) * lda + K) * 2 <= 0xffffffffL && (long(N - 1) * ldb + K) * 2 <= 0xffffffffL &&
         (uintptr_t)A % 16 == 0 && (uintptr_t)Bt % 16 == 0 && lda % 8 == 0 && ldb % 8 == 0;
}

hipError_t gemm_pipe(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                     long sa, long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st) {
  if (M <= 0 || N <= 0 || batch <= 0) return hipSuccess;
  if (!gemm_pipe_ok(dt, A, Bt, M, N, K, lda, ldb, sa, sb)) return hipErrorInvalidValue;
  if (dt == BF16) return launch_dt<BF16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile, st);
  return launch_dt<F16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile, st);
}

}  // namespace mh
