// MFMA GEMM for gfx950: C[M,N] = A[M,K] * Bt[N,K]^T with a fused epilogue.
//
// This is the compute behind BackendBlasCapability::matmul / batched_matmul
// (reference src/core/backend.hpp:250-260, CPU semantics in
// src/backend/cpu_backend.hpp:334-414) and behind nn::Linear
// (src/nn/linear.hpp:28-34: y = x.matmul(W) + b, W stored [in, out]).
//
// Design (CDNA4-first, not derived from any CUDA kernel):
//   * 256 threads = 4 wave64s in a WGM x WGN grid; block tile BM x BN; every
//     K step stages a 128-byte-deep slab of A and Bt through LDS (64 bf16/fp16
//     or 32 fp32 values per row), double buffered, one barrier per step.
//   * Both operands are K-contiguous in LDS, split in 16-byte chunks with an
//     XOR swizzle (chunk c of row r lives at c ^ (r & 7)) so the 16-byte
//     fragment reads of 8 consecutive rows hit distinct banks.
//   * 16-bit types use v_mfma_f32_16x16x32_{bf16,f16}; fp32 uses four
//     v_mfma_f32_16x16x4_f32 per 16-byte chunk (full fp32 precision).
//   * Operands are fed "swapped" (Bt fragment as the MFMA A operand) so each
//     lane ends up holding 4 consecutive output columns of one row, which
//     makes the epilogue a single 8/16-byte store per fragment.
//   * Epilogue reproduces the reference's per-op rounding chain in registers:
//     round(matmul) -> round(+bias) -> activation -> round(+residual), with
//     GELU as the reference's three rounded ops x*sigmoid(round(x*c))
//     (src/nn/activations.hpp:31-38).  Optional head-split output writes
//     q/k/v straight into the [B,H,T,hd] layout that MultiHeadAttention
//     produces with permute+contiguous (src/nn/attention.hpp:51-62).
//   * Grid order: workgroups are dealt round-robin to the 8 XCDs; the tile
//     index is remapped so each XCD walks a contiguous band of tiles, then
//     grouped along M so consecutive tiles share Bt panels in that XCD's L2.
#include "mh_common.hpp"
#include "mh_kernels.hpp"
#include "gemm_common.hpp"

#include <cstdlib>
#include <stdexcept>
#include <string>

namespace mh {

namespace {



// Load one 16-byte chunk (kElems values starting at column k of row `row`),
// zero-filling whatever lies outside [0,rows) x [0,K).
template <int DT, bool VEC>
__device__ __forceinline__ uint4 load_chunk(const typename Store<DT>::T *__restrict__ p, long ld, int row,
                                            int rows, int k, int K) {
  constexpr int E = Mfma<DT>::kElems;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row >= rows) return v;
  const typename Store<DT>::T *src = p + long(row) * ld + k;
  if (VEC && k + E <= K) return *reinterpret_cast<const uint4 *>(src);
  typename Store<DT>::T tmp[E];
#pragma unroll
  for (int e = 0; e < E; ++e) tmp[e] = (k + e < K) ? src[e] : typename Store<DT>::T(0);
  __builtin_memcpy(&v, tmp, 16);
  return v;
}

// Chunk at the K tail: values at or beyond K read as zero.
template <int DT, bool VEC>
__device__ __forceinline__ uint4 load_tail(const typename Store<DT>::T *__restrict__ src, int k, int K) {
  typedef typename Store<DT>::T T;
  constexpr int E = Mfma<DT>::kElems;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (VEC && k + E <= K) return *reinterpret_cast<const uint4 *>(src);
  T tmp[E];
#pragma unroll
  for (int e = 0; e < E; ++e) tmp[e] = (k + e < K) ? src[e] : T(0);
  __builtin_memcpy(&v, tmp, 16);
  return v;
}

// im2col chunk from an NHWC activation: GEMM row m = output pixel
// (b, oh, ow), column k = (kh*kW + kw)*iC + ic.  Rows are pre-decoded into
// (pixel base, ih0, iw0) once per thread.
template <int DT, bool VEC>
__device__ __forceinline__ uint4 load_im2col(const typename Store<DT>::T *__restrict__ x, const ConvArgs &cv, bool rowok,
                                             long pixbase, int ih0, int iw0, int k, int K) {
  typedef typename Store<DT>::T T;
  constexpr int E = Mfma<DT>::kElems;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (!rowok) return v;
  const int kk = k / cv.iC, ic0 = k - kk * cv.iC;
  if (VEC && k + E <= K) {
    const int kh = kk / cv.kW, kw = kk - kh * cv.kW;
    const int ih = ih0 + kh, iw = iw0 + kw;
    if (ih >= 0 && ih < cv.iH && iw >= 0 && iw < cv.iW)
      v = *reinterpret_cast<const uint4 *>(x + (pixbase + long(ih) * cv.iW + iw) * cv.ldx + ic0);
    return v;
  }
  T tmp[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    tmp[e] = T(0);
    const int ke = k + e;
    if (ke < K) {
      const int q = ke / cv.iC, ic = ke - q * cv.iC;
      const int kh = q / cv.kW, kw = q - kh * cv.kW;
      const int ih = ih0 + kh, iw = iw0 + kw;
      if (ih >= 0 && ih < cv.iH && iw >= 0 && iw < cv.iW) tmp[e] = x[(pixbase + long(ih) * cv.iW + iw) * cv.ldx + ic];
    }
  }
  __builtin_memcpy(&v, tmp, 16);
  return v;
}

template <int DT, int BM, int BN, int WGM, int WGN, bool VEC, bool CONV>
__global__ void __launch_bounds__(WGM * WGN * 64)
gemm_nt_kernel(const typename Store<DT>::T *__restrict__ A, const typename Store<DT>::T *__restrict__ Bt,
               int M, int N, int K, long lda, long ldb, long sa, long sb, long sc, EpiArgs ep, ConvArgs cv) {
  typedef typename Store<DT>::T T;
  constexpr int E = Mfma<DT>::kElems;
  constexpr int BK = 8 * E;  // 8 chunks of 16 bytes per row
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  constexpr int kThreads = WGM * WGN * 64;
  constexpr int ACH = BM * 8 / kThreads, BCH = BN * 8 / kThreads;
  static_assert(ACH >= 1 && BCH >= 1, "tile too small");

  extern __shared__ uint4 smem[];
  uint4 *As = smem;                 // [2][BM*8]
  uint4 *Bs = smem + 2 * BM * 8;    // [2][BN*8]

  // ---- tile scheduling (XCD band + group-M swizzle) ----
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int ntiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  constexpr int GROUP = 8;
  const int group_span = GROUP * tiles_n;
  const int gid = pid / group_span;
  const int first_m = gid * GROUP;
  const int gsize = min(tiles_m - first_m, GROUP);
  const int tm = first_m + (pid % group_span) % gsize;
  const int tn = (pid % group_span) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const int z = blockIdx.z;
  A += z * sa;
  Bt += z * sb;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;

  uint4 ra[ACH], rb[BCH];
  // Per-thread source rows are fixed for the whole K loop.  Rows past M / N
  // are clamped to the last valid row: they only feed output rows/columns
  // that are never stored, so no per-load branch is needed.
  const typename Store<DT>::T *arow[CONV ? 1 : ACH];
  const typename Store<DT>::T *brow[BCH];
  long pixbase[CONV ? ACH : 1];
  int ih0[CONV ? ACH : 1], iw0[CONV ? ACH : 1];
  bool rowok[CONV ? ACH : 1];
  const int cidx = (tid & 7) * E;  // column of this thread's chunk in a slab
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int m = m0 + ((tid + i * kThreads) >> 3);
    if (CONV) {
      const int ow = m % cv.oW, t2 = m / cv.oW, oh = t2 % cv.oH, b = t2 / cv.oH;
      pixbase[i] = long(b) * cv.iH * cv.iW;
      ih0[i] = oh * cv.s - cv.p;
      iw0[i] = ow * cv.s - cv.p;
      rowok[i] = m < M;
    } else {
      arow[i] = A + long(min(m, M - 1)) * lda + cidx;
    }
  }
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int n = n0 + ((tid + i * kThreads) >> 3);
    brow[i] = Bt + long(min(n, N - 1)) * ldb + cidx;
  }

#define MH_GLOAD(k0)                                                                                   \
  {                                                                                                    \
    const bool kfull = VEC && ((k0) + BK <= K);                                                        \
    if (kfull) {                                                                                       \
      _Pragma("unroll") for (int i = 0; i < ACH; ++i) {                                                \
        if (CONV) ra[i] = load_im2col<DT, true>(A, cv, rowok[i], pixbase[i], ih0[i], iw0[i], (k0) + cidx, K); \
        else ra[i] = *reinterpret_cast<const uint4 *>(arow[i] + (k0));                                 \
      }                                                                                                \
      _Pragma("unroll") for (int i = 0; i < BCH; ++i) rb[i] = *reinterpret_cast<const uint4 *>(brow[i] + (k0)); \
    } else {                                                                                           \
      _Pragma("unroll") for (int i = 0; i < ACH; ++i) {                                                \
        if (CONV) ra[i] = load_im2col<DT, VEC>(A, cv, rowok[i], pixbase[i], ih0[i], iw0[i], (k0) + cidx, K); \
        else ra[i] = load_tail<DT, VEC>(arow[i] + (k0), (k0) + cidx, K);                               \
      }                                                                                                \
      _Pragma("unroll") for (int i = 0; i < BCH; ++i) rb[i] = load_tail<DT, VEC>(brow[i] + (k0), (k0) + cidx, K); \
    }                                                                                                  \
  }
#define MH_SSTORE(buf)                                                                                 \
  {                                                                                                    \
    uint4 *as_ = As + (buf) * BM * 8, *bs_ = Bs + (buf) * BN * 8;                                      \
    _Pragma("unroll") for (int i = 0; i < ACH; ++i) {                                                  \
      const int id = tid + i * kThreads, r = id >> 3, c = id & 7;                                      \
      as_[r * 8 + (c ^ (r & 7))] = ra[i];                                                              \
    }                                                                                                  \
    _Pragma("unroll") for (int i = 0; i < BCH; ++i) {                                                  \
      const int id = tid + i * kThreads, r = id >> 3, c = id & 7;                                      \
      bs_[r * 8 + (c ^ (r & 7))] = rb[i];                                                              \
    }                                                                                                  \
  }

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = (K + BK - 1) / BK;
  MH_GLOAD(0);
  MH_SSTORE(0);
  __syncthreads();

  const int lrow = lane & 15, lgrp = lane >> 4;
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) MH_GLOAD((kt + 1) * BK);
    const uint4 *as = As + buf * BM * 8, *bs = Bs + buf * BN * 8;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 4 + lgrp;
      uint4 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * WTM + i * 16 + lrow;
        af[i] = as[r * 8 + (c ^ (r & 7))];
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int r = wn * WTN + j * 16 + lrow;
        bf[j] = bs[r * 8 + (c ^ (r & 7))];
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Mfma<DT>::step(acc[i][j], bf[j], af[i]);
    }
    if (kt + 1 < KT) MH_SSTORE(buf ^ 1);
    __syncthreads();
  }
#undef MH_GLOAD
#undef MH_SSTORE

  // ---- epilogue ----
  // the batch slice offset is passed separately: a modified copy of the
  // epilogue arguments would live in private memory
  store_tile<DT, BM, BN, WTM, WTN, FM, FN, WGM * WGN>(acc, reinterpret_cast<float *>(smem), ep, m0 + wm * WTM,
                                                     n0 + wn * WTN, M, N, wave, lane,
                                                     ep.mode == EPI_ROWMAJOR ? z * sc : 0);
}

template <int DT, int BM, int BN, int WGM, int WGN, bool VEC, bool CONV>
void launch_one(dim3 grid, size_t lds, hipStream_t st, const void *A, const void *Bt, int M, int N, int K, long lda,
                long ldb, long sa, long sb, long sc, const EpiArgs &ep, const ConvArgs &cv) {
  typedef typename Store<DT>::T T;
  auto kfn = gemm_nt_kernel<DT, BM, BN, WGM, WGN, VEC, CONV>;
  // Raise the dynamic-LDS limit once per instantiation (first launch happens
  // outside stream capture: engines run one eager forward before capturing).
  static bool lds_attr_set = false;
  if (lds > 65536 && !lds_attr_set) {
    (void)hipFuncSetAttribute((const void *)kfn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    lds_attr_set = true;
  }
  hipLaunchKernelGGL(kfn, grid, dim3(WGM * WGN * 64), lds, st, (const T *)A, (const T *)Bt, M, N, K, lda, ldb, sa, sb, sc,
                     ep, cv);
}

template <int DT, int BM, int BN, int WGM, int WGN>
hipError_t launch_cfg(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                      long sa, long sb, long sc, const EpiArgs &ep, const ConvArgs *cv, hipStream_t st) {
  constexpr int E = Mfma<DT>::kElems;
  const size_t lds = size_t(2) * (BM + BN) * 8 * 16;
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  bool vec = (ldb % E == 0) && (sb % E == 0) && ((uintptr_t)A % 16 == 0) && ((uintptr_t)Bt % 16 == 0);
  if (cv) vec = vec && (cv->iC % E == 0) && (cv->ldx % E == 0);
  else vec = vec && (lda % E == 0) && (sa % E == 0);
  dim3 grid(tiles, 1, batch);
  const ConvArgs none{};
  // Instantiated variants: the aligned (VEC) path for every tile; the
  // unaligned path only for the 64x64 tile (host falls back to it); the conv
  // loader for tiles up to 256x128.
  constexpr bool kSmall = (BM == 64 && BN == 64);
  if (cv) {
    if constexpr (BM * BN <= 256 * 128 && WGM * WGN == 4) {
      if (vec) launch_one<DT, BM, BN, WGM, WGN, true, true>(grid, lds, st, A, Bt, M, N, K, lda, ldb, sa, sb, sc, ep, *cv);
      else if constexpr (kSmall) launch_one<DT, BM, BN, WGM, WGN, false, true>(grid, lds, st, A, Bt, M, N, K, lda, ldb, sa, sb, sc, ep, *cv);
      else return hipErrorInvalidValue;
    } else {
      return hipErrorInvalidValue;
    }
  } else {
    if (vec) launch_one<DT, BM, BN, WGM, WGN, true, false>(grid, lds, st, A, Bt, M, N, K, lda, ldb, sa, sb, sc, ep, none);
    else if constexpr (kSmall) launch_one<DT, BM, BN, WGM, WGN, false, false>(grid, lds, st, A, Bt, M, N, K, lda, ldb, sa, sb, sc, ep, none);
    else return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Choose the block tile that minimises (waves of tiles) x (tile cost) on 256
// CUs, preferring larger tiles for operand reuse when the wave count ties.
template <int DT>
hipError_t launch_dt(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
                     long sb, long sc, const EpiArgs &ep, const ConvArgs *cv, int tile_hint, hipStream_t st) {
  struct Cand { int bm, bn; double cost; };
  const int kCU = 256;
  Cand cands[5] = {{256, 256, 4.0}, {256, 128, 2.0}, {128, 128, 1.0}, {128, 64, 0.55}, {64, 64, 0.3}};
  int best = 2;
  if (tile_hint >= 0 && tile_hint < 8) {
    best = tile_hint;
  } else if (DT != F32 && !cv && long((M + 255) / 256) * ((N + 255) / 256) * batch >= 1024) {
    best = 7;  // 256x256, 8 waves: measured best for large GEMMs (LM head)
  } else if (DT != F32 && !cv && long((M + 127) / 128) * ((N + 127) / 128) * batch >= 128) {
    best = 2;  // 128x128, two blocks per CU: measured best for the layer GEMMs
  } else {
    double best_t = 1e30;
    for (int c = 0; c < 5; ++c) {
      const long tiles = long((M + cands[c].bm - 1) / cands[c].bm) * ((N + cands[c].bn - 1) / cands[c].bn) * batch;
      const long waves = (tiles + kCU - 1) / kCU;
      // per-tile cost grows with the tile area, discounted for better reuse
      const double t = double(waves) * cands[c].cost;
      if (t < best_t * 0.999) { best_t = t; best = c; }
    }
  }
  constexpr int E = Mfma<DT>::kElems;
  bool vec = (ldb % E == 0) && (sb % E == 0) && ((uintptr_t)A % 16 == 0) && ((uintptr_t)Bt % 16 == 0);
  if (cv) vec = vec && (cv->iC % E == 0) && (cv->ldx % E == 0);
  else vec = vec && (lda % E == 0) && (sa % E == 0);
  if (!vec) best = 4;
  if ((cv || DT == F32) && best == 0) best = 1;  // 256x256 only for 16-bit plain GEMMs
  if ((cv || DT == F32) && best >= 5) best = 2;  // 8-wave tiles only for 16-bit plain GEMMs
  switch (best) {
  case 0: return launch_cfg<DT, 256, 256, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, cv, st);
  case 1: return launch_cfg<DT, 256, 128, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, cv, st);
  case 2: return launch_cfg<DT, 128, 128, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, cv, st);
  case 3: return launch_cfg<DT, 128, 64, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, cv, st);
  case 5:
    if constexpr (DT != F32) return launch_cfg<DT, 256, 128, 4, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, cv, st);
    return hipErrorInvalidValue;
  case 6:
    if constexpr (DT != F32) return launch_cfg<DT, 128, 256, 2, 4>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, cv, st);
    return hipErrorInvalidValue;
  case 7:
    if constexpr (DT != F32) return launch_cfg<DT, 256, 256, 4, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, cv, st);
    return hipErrorInvalidValue;
  default: return launch_cfg<DT, 64, 64, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, cv, st);
  }
}

}  // namespace

hipError_t gemm_nt(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                   long sa, long sb, long sc, const EpiArgs &ep, int tile_hint, hipStream_t st) {
  if (M <= 0 || N <= 0 || batch <= 0) return hipSuccess;
  if (tile_hint < 0) {
    // MUNET_HIP_GEMM_TILE forces a kernel and block tile for tests and tuning:
    // 0-6 direct-to-LDS kernel, 100-107 general kernel, 200-203, 207-212,
    // 216, 217 and 219 pipelined kernel.  Read at every call so a process can
    // switch it between calls; any other code is an error.
    const char *force = std::getenv("MUNET_HIP_GEMM_TILE");
    if (force && *force) {
      tile_hint = std::atoi(force);
      const bool known = (tile_hint >= 0 && tile_hint <= 6) || (tile_hint >= 100 && tile_hint <= 107) ||
                         (tile_hint >= 200 && tile_hint <= 203) || (tile_hint >= 207 && tile_hint <= 212) ||
                         tile_hint == 216 || tile_hint == 217 || tile_hint == 219;
      if (!known)
        throw std::invalid_argument(std::string("MUNET_HIP_GEMM_TILE=") + force +
                                    " names no GEMM tile (0-6, 100-107, 200-203, 207-212, 216, 217, 219)");
    }
  }
  // <0: the pipelined 16-bit kernel when the operands allow it, else the
  // general kernel with an automatic tile.
  // A folded LayerNorm (stats_out / ln_stats) exists only in the pipelined
  // kernels: such a GEMM ignores a forced general-kernel tile, and fails when
  // its operands do not suit the pipelined kernels.
  // small fp32 products: one workgroup per 16x16 tile, K split over its waves
  if (tile_hint < 0 && gemm_skinny_ok(dt, A, Bt, M, N, K, lda, ldb, batch, ep))
    return gemm_skinny(A, Bt, M, N, K, lda, ldb, ep, st);
  const bool pipe = gemm_pipe_ok(dt, A, Bt, M, N, K, lda, ldb, sa, sb);
  const bool fold = ep.stats_out || ep.ln_stats;
  if (pipe && (tile_hint < 0 || tile_hint >= 200 || fold))
    return gemm_pipe(dt, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile_hint >= 200 ? tile_hint - 200 : -1, st);
  if (fold) return hipErrorInvalidValue;
  if (tile_hint >= 200) tile_hint = -1;
  if (tile_hint >= 0 && tile_hint < 100 && gemm_dma_ok(dt, A, Bt, K, lda, ldb, sa, sb))
    return gemm_dma(dt, A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile_hint, st);
  if (tile_hint >= 100) tile_hint -= 100;
  switch (dt) {
  case F32: return launch_dt<F32>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, nullptr, tile_hint, st);
  case F16: return launch_dt<F16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, nullptr, tile_hint, st);
  case BF16: return launch_dt<BF16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, nullptr, tile_hint, st);
  default: return hipErrorInvalidValue;
  }
}

// ---- split-K for small fp32 products --------------------------------------
// A product with few output tiles and a long K (the CNN's 32 x 4096 x 128
// Linear: two 64x64 tiles, 128 K steps each) leaves most CUs idle.  Split-K
// runs S <= 64 slices of K as a batch of partial products into an fp32
// workspace [S, M, N], then one kernel sums the slices in a fixed tree order
// (deterministic) and applies the epilogue chain.
int splitk_count(int dt, int M, int N, int K) {
  if (dt != F32 || M <= 0 || N <= 0 || K < 512) return 1;
  if (M <= 256 && long((M + 15) / 16) * ((N + 15) / 16) <= 1024 && K % 4 == 0 && K <= 2048) return 1;  // gemm_skinny
  const long tiles = long((M + 63) / 64) * ((N + 63) / 64);
  if (tiles >= 32) return 1;
  int best = 1;
  for (int S = 2; S <= 64; ++S) {
    if (tiles * S > 256) break;
    if (K % S || (K / S) % 4 || K / S < 64) continue;
    best = S;
  }
  return best;
}

namespace {
// One wave per output quad (m, n .. n+3): lane s loads slice s's partial quad
// (all slices in flight at once), a fixed xor-tree sums them, lane 0 applies
// the epilogue.
template <int DT>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float *__restrict__ ws, int S, int M, int N,
                                                             EpiArgs ep) {
  const int n4 = (N + 3) / 4, lane = threadIdx.x & 63;
  const long item = long(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (item >= long(M) * n4) return;
  const int m = int(item / n4), n = int(item - long(m) * n4) * 4;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (lane < S) {
    const float *p = ws + long(lane) * M * N + long(m) * N + n;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < N) v[e] = p[e];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += __shfl_xor(v[e], o, 64);
  if (lane == 0) epi_store4<DT>(ep, m, n, N, v, 0);
}
}  // namespace

hipError_t gemm_splitk(int dt, const void *A, const void *Bt, int M, int N, int K, int S, float *ws, const EpiArgs &ep,
                       hipStream_t st) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (dt != F32 || S < 1 || S > 64 || K % S || (K / S) % 4 || !ws || ep.mode != EPI_ROWMAJOR || ep.stats_out ||
      ep.ln_stats)
    return hipErrorInvalidValue;
  const int Kc = K / S;
  EpiArgs part;  // raw fp32 partial products, slice s at ws + s M N
  part.out = ws;
  part.ldc = N;
  hipError_t e = launch_dt<F32>(A, Bt, M, N, Kc, K, K, S, Kc, Kc, long(M) * N, part, nullptr, -1, st);
  if (e != hipSuccess) return e;
  const long items = long(M) * ((N + 3) / 4);
  hipLaunchKernelGGL(splitk_reduce_kernel<F32>, dim3(unsigned((items + 3) / 4)), dim3(256), 0, st, ws, S, M, N, ep);
  return hipGetLastError();
}

// ---- 1x1 convolution to a few output channels -------------------------------
// A 1x1 convolution to oC <= 8 channels (the UNet's output head: 64 -> 2) is
// a dot product per pixel: a matrix-core tile would waste all but oC of its
// columns.  One thread per output pixel reads its iC channels in 16-byte
// chunks (with NCH = iC / 8 known at compile time, all of them before the
// first product, so the chunks' latencies overlap), the weights sit in LDS as
// floats (every lane reads the same address), fp32 sums in channel order,
// then the epilogue chain.
namespace {
template <int DT, int NCH>
__global__ void __launch_bounds__(256) conv1x1_smalln_kernel(const uint16_t *__restrict__ x,
                                                              const uint16_t *__restrict__ w, int M, int iC, long ldx,
                                                              int oC, EpiArgs ep) {
  __shared__ float wl[8 * 512];
  for (int i = threadIdx.x; i < oC * iC; i += 256) wl[i] = Store<DT>::dec(w[i]);
  __syncthreads();
  const int m = blockIdx.x * 256 + threadIdx.x;
  if (m >= M) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const uint16_t *row = x + long(m) * ldx;
  auto chunk = [&](const uint4 q, int c0) {
    const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float xv = Store<DT>::dec(uint16_t(wd[e >> 1] >> (16 * (e & 1))));
#pragma unroll
      for (int o = 0; o < 8; ++o)
        if (o < oC) acc[o] = __fmaf_rn(xv, wl[o * iC + c0 + e], acc[o]);
    }
  };
  if constexpr (NCH > 0) {
    uint4 q[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) q[j] = *reinterpret_cast<const uint4 *>(row + 8 * j);
#pragma unroll
    for (int j = 0; j < NCH; ++j) chunk(q[j], 8 * j);
  } else {
    for (int c0 = 0; c0 < iC; c0 += 8) chunk(*reinterpret_cast<const uint4 *>(row + c0), c0);
  }
  float lo[4] = {acc[0], acc[1], acc[2], acc[3]}, hi[4] = {acc[4], acc[5], acc[6], acc[7]};
  epi_store4<DT>(ep, m, 0, oC, lo, 0);
  if (oC > 4) epi_store4<DT>(ep, m, 4, oC, hi, 0);
}

template <int DT>
hipError_t conv1x1_smalln(const uint16_t *x, const uint16_t *w, int M, int iC, long ldx, int oC, const EpiArgs &ep,
                          hipStream_t st) {
  const dim3 grid((M + 255) / 256), block(256);
  switch (iC) {
  case 32: hipLaunchKernelGGL((conv1x1_smalln_kernel<DT, 4>), grid, block, 0, st, x, w, M, iC, ldx, oC, ep); break;
  case 64: hipLaunchKernelGGL((conv1x1_smalln_kernel<DT, 8>), grid, block, 0, st, x, w, M, iC, ldx, oC, ep); break;
  case 128: hipLaunchKernelGGL((conv1x1_smalln_kernel<DT, 16>), grid, block, 0, st, x, w, M, iC, ldx, oC, ep); break;
  default: hipLaunchKernelGGL((conv1x1_smalln_kernel<DT, 0>), grid, block, 0, st, x, w, M, iC, ldx, oC, ep); break;
  }
  return hipGetLastError();
}

}  // namespace

// Implicit-GEMM convolution on an NHWC activation with OHWI-packed weights:
// M = B*oH*oW output pixels, N = oC, K = kH*kW*iC.  Output row m, column oc.
hipError_t conv_nhwc(int dt, const void *x, const void *w_ohwi, const ConvArgs &cv, int oC, const EpiArgs &ep,
                     int tile_hint, hipStream_t st) {
  const int M = cv.B * cv.oH * cv.oW, K = cv.kH * cv.kW * cv.iC;
  if (M <= 0 || oC <= 0) return hipSuccess;
  // 16-bit convolutions with whole 64-channel slabs run on the pipelined
  // kernel; MUNET_HIP_CONV_KERNEL=general (read per call) keeps this one
  const char *ck = std::getenv("MUNET_HIP_CONV_KERNEL");
  const bool general = ck && std::string(ck) == "general";
  if (tile_hint < 0 && !general && (dt == F16 || dt == BF16) && cv.kH == 1 && cv.kW == 1 && cv.s == 1 && cv.p == 0 &&
      oC <= 8 && cv.iC % 8 == 0 && cv.iC <= 512 && cv.ldx % 8 == 0 && (uintptr_t)x % 16 == 0 &&
      ep.mode == EPI_ROWMAJOR && !ep.resid) {
    return dt == F16 ? conv1x1_smalln<F16>((const uint16_t *)x, (const uint16_t *)w_ohwi, M, cv.iC, cv.ldx, oC, ep, st)
                     : conv1x1_smalln<BF16>((const uint16_t *)x, (const uint16_t *)w_ohwi, M, cv.iC, cv.ldx, oC, ep, st);
  }
  if (tile_hint < 0 && !general && gemm_pipe_conv_ok(dt, x, w_ohwi, cv))
    return gemm_pipe_conv(dt, x, w_ohwi, cv, oC, ep, st);
  switch (dt) {
  case F32: return launch_dt<F32>(x, w_ohwi, M, oC, K, 0, K, 1, 0, 0, 0, ep, &cv, tile_hint, st);
  case F16: return launch_dt<F16>(x, w_ohwi, M, oC, K, 0, K, 1, 0, 0, 0, ep, &cv, tile_hint, st);
  case BF16: return launch_dt<BF16>(x, w_ohwi, M, oC, K, 0, K, 1, 0, 0, 0, ep, &cv, tile_hint, st);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace mh
