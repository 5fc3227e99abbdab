// Direct-to-LDS, multi-stage MFMA GEMM for gfx950 (16-bit operands).
//
// Same contract and epilogue as gemm.hip (C = A[M,K] * Bt[N,K]^T, fused
// reference-rounding epilogue), specialised for the aligned case the engine
// produces (K % 64 == 0, 16-byte aligned rows):
//   * operands move global -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging, no ds_write): each wave instruction fills 1 KB of LDS = 8 rows
//     of a 128-byte K slab; lane l fetches the global chunk that the XOR
//     swizzle (chunk c of row r at c ^ (r & 7)) places at LDS slot l;
//   * S LDS stages with S-1 slabs in flight: at step k the wave waits for
//     slab k (vmcnt), one barrier, issues slab k+S-1 into the stage consumed
//     at step k-1, then computes slab k.  Stages are distinct LDS objects
//     indexed at compile time (the K loop is unrolled by S), so the compiler
//     can keep the loads in flight across the reads of other stages;
//   * the barrier is the raw s_barrier with compiler fences only: a
//     __syncthreads() release fence would wait for every load in flight.
#include "mh_common.hpp"
#include "mh_kernels.hpp"
#include "gemm_common.hpp"


namespace mh {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kThreadsD = 256;

__device__ __forceinline__ void barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt with only vmcnt(n) constrained (gfx9 encoding).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int BM, int BN, int S> struct DmaLds {
  uint4 a[S][BM * 8];
  uint4 b[S][BN * 8];
};

// Per-wave state of one output tile: DMA sources, stage buffers, MFMA loop.
// NW = WGM * WGN waves; each wave owns a (BM/WGM) x (BN/WGN) sub-tile.
template <int DT, int BM, int BN, int WGM, int WGN, int S> struct DmaTile {
  static constexpr int NW = WGM * WGN;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int FM = WTM / 16, FN = WTN / 16;
  static constexpr int ABLK = BM / 8 / NW, BBLK = BN / 8 / NW;  // 8-row DMA blocks per wave
  static constexpr int NDMA = ABLK + BBLK;                       // DMA instructions per slab per wave
  static_assert(ABLK * NW * 8 == BM && BBLK * NW * 8 == BN, "DMA split");
  static_assert(NDMA * (S - 1) < 64, "vmcnt range");
  static_assert(S >= 3, "fragment prefetch needs three stages");

  DmaLds<BM, BN, S> *sm;
  const uint16_t *asrc[ABLK];
  const uint16_t *bsrc[BBLK];
  int wave, wm, wn, lrow, lgrp, KT;
  f32x4 acc[FM][FN];

  template <int s> __device__ __forceinline__ void issue(int kt) {
    const int k0 = kt * 64;
#pragma unroll
    for (int i = 0; i < ABLK; ++i)
      __builtin_amdgcn_global_load_lds(asrc[i] + k0, (lds_void *)&sm->a[s][(wave * ABLK + i) * 64], 16, 0, 0);
#pragma unroll
    for (int i = 0; i < BBLK; ++i)
      __builtin_amdgcn_global_load_lds(bsrc[i] + k0, (lds_void *)&sm->b[s][(wave * BBLK + i) * 64], 16, 0, 0);
  }

  // fragments of k-step ks (32 of the slab's 64 K values) from stage s
  template <int s, int ks> __device__ __forceinline__ void frags(uint4 (&af)[FM], uint4 (&bf)[FN]) {
    const uint4 *as = sm->a[s], *bs = sm->b[s];
    const int c = ks * 4 + lgrp;
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
  }

  __device__ __forceinline__ void mma(const uint4 (&af)[FM], const uint4 (&bf)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) Mfma<DT>::step(acc[i][j], bf[j], af[i]);
  }

  // Wait until slab `need` has landed given that slabs up to `issued` were
  // issued (at most S-2 slabs beyond it can be in flight).
  __device__ __forceinline__ void wait_slab(int need, int issued) {
    const int ahead = issued - need;
    if (ahead >= 2 && S >= 4) wait_vmcnt<NDMA * 2 < 64 ? NDMA * 2 : 0>();
    else if (ahead >= 1) wait_vmcnt<NDMA>();
    else wait_vmcnt<0>();
  }

  // Slab kt in stage s; F0 holds its first-half fragments on entry and the
  // next slab's first-half fragments on exit.
  template <int s> __device__ __forceinline__ void step(int kt, uint4 (&f0a)[FM], uint4 (&f0b)[FN]) {
    constexpr int snext = (s + 1) % S, srefill = (s + S - 1) % S;
    uint4 f1a[FM], f1b[FN];
    this->template frags<s, 1>(f1a, f1b);  // in flight under the first half's MFMAs
    __builtin_amdgcn_sched_barrier(0);
    mma(f0a, f0b);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < KT) {
      wait_slab(kt + 1, min(kt + S - 2, KT - 1));
      barrier_nofence();  // slab kt+1 visible; every wave is done with stage srefill
      if (kt + S - 1 < KT) this->template issue<srefill>(kt + S - 1);
      this->template frags<snext, 0>(f0a, f0b);  // in flight under the second half
    }
    __builtin_amdgcn_sched_barrier(0);
    mma(f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);
  }
};

template <int DT, int BM, int BN, int WGM, int WGN, int S>
__global__ void __launch_bounds__(WGM * WGN * 64)
gemm_dma_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ Bt, int M, int N, int K, long lda,
                long ldb, long sa, long sb, long sc, EpiArgs ep) {
  // The body uses the LDS-DMA builtin and address-space-3 pointers, which only
  // exist in the device compilation pass; the host pass needs just the stub.
#if defined(__HIP_DEVICE_COMPILE__)
  typedef typename Store<DT>::T T;
  typedef DmaTile<DT, BM, BN, WGM, WGN, S> Tile;
  __shared__ DmaLds<BM, BN, S> sm;

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

  const int tid = threadIdx.x, lane = tid & 63;
  Tile t;
  t.sm = &sm;
  t.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  t.wm = t.wave / WGN;
  t.wn = t.wave % WGN;
  t.lrow = lane & 15;
  t.lgrp = lane >> 4;
  t.KT = K / 64;
  // lane l of a DMA fetches block row l/8, global chunk (l%8) ^ (l/8): the
  // chunk the swizzle stores at LDS slot l
  const int lr = lane >> 3, lc = (lane & 7) ^ lr;
#pragma unroll
  for (int i = 0; i < Tile::ABLK; ++i) {
    const int row = m0 + (t.wave * Tile::ABLK + i) * 8 + lr;
    t.asrc[i] = A + long(min(row, M - 1)) * lda + lc * 8;
  }
#pragma unroll
  for (int i = 0; i < Tile::BBLK; ++i) {
    const int row = n0 + (t.wave * Tile::BBLK + i) * 8 + lr;
    t.bsrc[i] = Bt + long(min(row, N - 1)) * ldb + lc * 8;
  }
#pragma unroll
  for (int i = 0; i < Tile::FM; ++i)
#pragma unroll
    for (int j = 0; j < Tile::FN; ++j) t.acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = t.KT;
  // prologue: slabs 0 .. S-2 in flight, then slab 0's first-half fragments
  t.template issue<0>(0);
  if (1 < KT) t.template issue<1>(1);
  if constexpr (S > 3) {
    if (2 < KT) t.template issue<2>(2);
  }
  t.wait_slab(0, min(S - 2, KT - 1));
  barrier_nofence();
  uint4 f0a[Tile::FM], f0b[Tile::FN];
  t.template frags<0, 0>(f0a, f0b);
  for (int kt = 0; kt < KT; kt += S) {
    t.template step<0>(kt, f0a, f0b);
    if (kt + 1 < KT) t.template step<1>(kt + 1, f0a, f0b);
    if (kt + 2 < KT) t.template step<2>(kt + 2, f0a, f0b);
    if constexpr (S > 3) {
      if (kt + 3 < KT) t.template step<3>(kt + 3, f0a, f0b);
    }
  }
  barrier_nofence();  // every wave done reading the stages before they are reused

  store_tile<DT, BM, BN, Tile::WTM, Tile::WTN, Tile::FM, Tile::FN, Tile::NW>(
      t.acc, reinterpret_cast<float *>(&sm), ep, m0 + t.wm * Tile::WTM, n0 + t.wn * Tile::WTN, M, N, t.wave, lane,
      ep.mode == EPI_ROWMAJOR ? z * sc : 0);
#endif
}

template <int DT, int BM, int BN, int WGM, int WGN, int S>
hipError_t launch_dma(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
                      long sb, long sc, const EpiArgs &ep, hipStream_t st) {
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_dma_kernel<DT, BM, BN, WGM, WGN, S>), dim3(tiles, 1, batch), dim3(WGM * WGN * 64), 0, st,
                     (const uint16_t *)A, (const uint16_t *)Bt, M, N, K, lda, ldb, sa, sb, sc, ep);
  return hipGetLastError();
}

template <int DT>
hipError_t dma_dt(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa, long sb,
                  long sc, const EpiArgs &ep, int tile, hipStream_t st) {
  switch (tile) {
  case 0: return launch_dma<DT, 256, 128, 2, 2, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  case 1: return launch_dma<DT, 128, 256, 2, 2, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  case 2: return launch_dma<DT, 128, 128, 2, 2, 4>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  case 3: return launch_dma<DT, 128, 128, 2, 2, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  case 4: return launch_dma<DT, 256, 128, 4, 2, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  case 5: return launch_dma<DT, 128, 256, 2, 4, 3>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  default: return launch_dma<DT, 128, 64, 2, 2, 4>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st);
  }
}

}  // namespace

bool gemm_dma_ok(int dt, const void *A, const void *Bt, int K, long lda, long ldb, long sa, long sb) {
  return (dt == F16 || dt == BF16) && K % 64 == 0 && K > 0 && lda % 8 == 0 && ldb % 8 == 0 && sa % 8 == 0 &&
         sb % 8 == 0 && ((uintptr_t)A % 16 == 0) && ((uintptr_t)Bt % 16 == 0);
}

hipError_t gemm_dma(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
                    long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st) {
  if (dt == BF16) return dma_dt<BF16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile, st);
  return dma_dt<F16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile, st);
}

}  // namespace mh
