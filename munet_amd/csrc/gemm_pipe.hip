// Pipelined 16-bit MFMA GEMM (gemm_pipe.hpp): the general epilogue program
// on block tiles up to 128 rows, with the accumulators in ordinary VGPRs
// (built with -amdgpu-mfma-vgpr-form, see build.py), and the dispatcher that
// picks the block tile and the epilogue program.  The fixed bf16 programs
// are instantiated in gemm_pipe_fixed_*.hip, the eight-wave tiles in
// gemm_pipe_wide.hip.
#include <algorithm>
#include "gemm_pipe.hpp"

namespace mh {

namespace {

// Width of one wave's tile (columns) for each tile code.
int pipe_wave_cols(int tile) {
  switch (tile) {
  case 0: case 7: case 9: return 64;
  case 3: case 8: case 10: case 11: case 17: return 48;
  case 16: return 96;
  case 19: return 144;
  default: return 32;  // 1 (128x64), 2 (64x64), 12 (128x64)
  }
}

// Automatic block tile, measured on MI355X inside the decoder forward
// (K = 768 / 3072, M = 4096):
//  * M tiling evenly by 256 and N by 192 into 232..256 tiles (FFN up: 256):
//    direct-to-LDS 256x192 with eight waves, one workgroup per CU (FFN up
//    33.1 -> 31.1 us; QKV, 192 tiles, 28.3 -> 29.5 us, so it stays below);
//  * M tiling by 128 and N by 288 into 232..256 tiles (QKV, 4096 x 2304):
//    direct-to-LDS 128x288, eight waves of 32x144, one workgroup per CU
//    (forward 1.620 -> 1.609 ms against the register-staged 128x96, whose
//    768 tiles take three rounds of two workgroups per CU);
//  * N tiling evenly by 96 with at most one tile per CU (N = 768: FFN down,
//    attention out-projection): direct-to-LDS 128x96, 4 stages, eight waves
//    (one workgroup per CU, so deep stages and two waves per SIMD hide the
//    memory latency; out-projection 13.9 -> 12.9 us against four waves);
//  * otherwise register-staged: 128x128 when N tiles evenly by 128 and there
//    are >= 2.5 tiles per CU (FFN up, LM head), 128x96 when N tiles evenly by
//    96 (QKV), else 128x128 / 128x64 / 64x64 by tile count.
// (The vocabulary head, a non-temporal output, takes direct-to-LDS 128x128
// with two stages: see launch_dt.)
int auto_tile(bool dma, int M, int N, int K, int batch) {
  const long t128 = long((M + 127) / 128) * ((N + 127) / 128) * batch;
  const long t96 = long((M + 127) / 128) * ((N + 95) / 96) * batch;
  const long t64 = long((M + 127) / 128) * ((N + 63) / 64) * batch;
  const long t192w = long(M / 256) * (N / 192) * batch;
  if (dma && M % 256 == 0 && N % 192 == 0 && t192w >= 232 && t192w <= 256) return 16;
  const long t288 = long(M / 128) * (N / 288) * batch;
  if (dma && M % 128 == 0 && N % 288 == 0 && t288 >= 232 && t288 <= 256) return 19;
  if (dma && N % 96 == 0 && t96 <= 256) return 17;
  if (N % 128 == 0 && t128 >= 640) return 0;
  if (N % 96 == 0) return 3;
  return (t128 >= 640 || (K >= 2048 && t128 >= 128)) ? 0 : (t64 >= 256 ? 1 : 2);
}

// The tiles with fixed epilogue programs (gemm_pipe_fixed_*.hip).
bool fixed_tile(int tile) {
  return (tile >= 0 && tile <= 3) || tile == 8 || tile == 9 || tile == 16 || tile == 17 || tile == 19;
}

// The epilogue program for these arguments: a fixed program for the
// combinations the engine emits (bf16, 8-byte aligned destination, bias
// after the matmul rounding), else PK_GENERAL; -1 for a folded LayerNorm
// outside the fixed programs (it has no general form).
int pipe_kind(int dt, int N, int batch, long sc, const EpiArgs &ep) {
  const bool fold = ep.ln_stats || ep.stats_out;
  const bool fast = (dt == BF16 || dt == F16) && N % 4 == 0 && ep.mode != EPI_CONVT && (!ep.resid || (ep.ldr & 3) == 0);
  const bool al8 = ep.mode == EPI_HEADSPLIT
                       ? (ep.hd & 3) == 0 && ((uintptr_t)ep.outs[0] & 7) == 0 && ((uintptr_t)ep.outs[1] & 7) == 0 &&
                             ((uintptr_t)ep.outs[2] & 7) == 0
                       : ((uintptr_t)ep.out & 7) == 0 && (ep.ldc & 3) == 0 && (batch == 1 || (sc & 3) == 0);
  if (!fast || !al8 || (ep.bias && ep.bias_first)) return fold ? -1 : PK_GENERAL;
  const bool hb = ep.bias != nullptr, hr = ep.resid != nullptr;
  if (fold && dt != BF16) return -1;  // the folded LayerNorm programs are bf16 only
  if (ep.ln_stats) {
    if (ep.stats_out || !hb || hr) return -1;
    return ep.act == ACT_NONE ? PK_LN_BIAS : ep.act == ACT_GELU ? PK_LN_BIAS_GELU : -1;
  }
  if (ep.stats_out) return hb && hr && ep.act == ACT_NONE ? PK_BIAS_RESID_ST : -1;
  if (ep.act == ACT_NONE) return !hb && !hr ? PK_PLAIN : hb && !hr ? PK_BIAS : hb && hr ? PK_BIAS_RESID : PK_GENERAL;
  return ep.act == ACT_GELU && hb && !hr ? PK_BIAS_GELU : PK_GENERAL;
}

template <int DT>
hipError_t launch_dt(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
                     long sb, long sc, const EpiArgs &ep, int tile, int kind, hipStream_t st) {
  const bool dma = gemm_pipe_dma_ok(A, Bt, M, N, K, lda, ldb);
  // a folded LayerNorm exists only in the fixed programs: a forced tile
  // without the program takes the automatic choice
  // a large streamed output (the vocabulary head): direct-to-LDS 128x128,
  // two stages (with the late wait for the next slab: forward 1.506 ->
  // 1.491 ms against the register-staged 128x128, 1.497 on the 256x256 tile)
  if (tile < 0 && kind == PK_BIAS_NT && dma) tile = 9;
  // a transposed convolution (K = iC <= 512, scattered output rows): the
  // register-staged 64x64, whose many small workgroups hide the load and
  // store latencies of its few K steps (UNet fp16: up2 14.7 -> 11.1 us, up1
  // 11.5 -> 10.4, up0 19.1 -> 15.1 against 128x64; the direct-to-LDS 128x128
  // 20-31 us)
  if (tile < 0 && ep.mode == EPI_CONVT) tile = 2;
  if (tile < 0 || (kind >= PK_LN_BIAS && !fixed_tile(tile))) tile = auto_tile(dma, M, N, K, batch);
  if (tile >= 7 && !dma) tile = 0;
  if (tile == 19 && (M % 128 || N % 288)) tile = auto_tile(dma, M, N, K, batch);
  // LayerNorm partials of stats_cols columns need wave tiles that cover whole
  // groups: move to the nearest tile whose wave-tile width is a multiple
  if (ep.stats_out && pipe_wave_cols(tile) % ep.stats_cols)
    tile = ep.stats_cols == 48 ? (dma ? 8 : 3) : ep.stats_cols == 64 ? (dma ? 9 : 0) : 2;
  if (tile == 16 || tile == 17 || tile == 19)
    return gemm_pipe_wide(DT, kind, tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  if (kind > PK_GENERAL && fixed_tile(tile))
    return tile <= 3 ? gemm_pipe_fixed_staged(DT, kind, tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st)
                     : gemm_pipe_fixed_dma(DT, kind, tile, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
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
  const int kind = pipe_kind(dt, N, batch, sc, ep);
  if (kind < 0) return hipErrorInvalidValue;
  // the folded-LayerNorm terms (fixed programs only)
  if (ep.stats_out || ep.ln_stats) {
    const bool cols_ok = ep.stats_cols == 16 || ep.stats_cols == 32 || ep.stats_cols == 48 || ep.stats_cols == 64;
    if ((ep.stats_out && (!cols_ok || N % ep.stats_cols || ep.mode != EPI_ROWMAJOR || batch != 1)) ||
        (ep.ln_stats && (ep.ln_parts <= 0 || ep.ln_parts > 64 || ep.ln_cols <= 0 || K != ep.ln_cols * ep.ln_parts ||
                         !ep.ln_cs || !ep.ln_bw || batch != 1)))
      return hipErrorInvalidValue;
  }
  // tile enumeration: column groups once W is at least half of A (measured
  // on the decoder's forward, cold weights: QKV and FFN up -2.5 to -3.5 us
  // with 8 columns, the vocabulary head -45 us with 16; FFN down and
  // out-proj, whose A is 4-5x W, stay on row groups); MUNET_HIP_XCD_GN
  // overrides it for every GEMM
  const int kd = kind == PK_BIAS && ep.stream_out ? PK_BIAS_NT : kind;
  EpiArgs e = ep;
  e.xcd_gn = 2L * N >= M ? (N >= 4L * M ? 16 : 8) : 0;
  if (const char *gn = std::getenv("MUNET_HIP_XCD_GN")) e.xcd_gn = std::max(0, std::atoi(gn));
  if (e.pf_bytes <= 0 || e.pf_bytes > (16L << 20)) e.pf = nullptr;
  if (dt == BF16) return launch_dt<BF16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, e, tile, kd, st);
  return launch_dt<F16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, e, tile, kd, st);
}

}  // namespace mh
