// Pipelined 16-bit MFMA GEMM for gfx950: C[M,N] = A[M,K] * Bt[N,K]^T with the
// fused epilogue of gemm_common.hpp (the reference semantics are those of
// BackendBlasCapability::matmul and nn::Linear, src/core/backend.hpp:250-260,
// src/nn/linear.hpp:28-34).
//
// The hot path of the decoder's Linear layers (bf16/fp16, 16-byte aligned
// K-contiguous operands).  Differences from the general kernel in gemm.hip:
//   * each 64-wide K step runs in two phases split by the one barrier of the
//     step.  Phase A multiplies the first 32-wide K half (fragments already in
//     registers) while it reads the second half's fragments, stores the next
//     slab (staged in registers) to the other LDS buffer and requests the
//     slab after it from memory; phase B multiplies the second half while it
//     reads the next slab's first-half fragments.  __builtin_amdgcn_
//     sched_group_barrier pins that interleaving, one memory operation after
//     each MFMA, so every LDS and global access is covered by MFMA work of the
//     same wave;
//   * the K loop has no conditional loads: a K % 64 remainder is taken as a
//     short (zero-padded) first slab, every later slab is whole, and the loads
//     of the last step re-read the last slab, so the staging registers never
//     merge values from different control paths;
//   * global loads use 32-bit per-thread offsets from slab base pointers that
//     advance one slab per step;
//   * staging registers and LDS use native clang vector types (no struct
//     copies through private memory);
//   * the epilogue runs on each accumulator fragment in registers (no LDS
//     staging): lane (r, g) of a 16x16 fragment owns row r, columns 4g..4g+3;
//     its bias and residual loads are issued before the K loop.
// Built with MFMA results in ordinary VGPRs (see build.py).
#include "mh_common.hpp"
#include "mh_kernels.hpp"
#include "gemm_common.hpp"

namespace mh {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte load through a global-address-space pointer.  The loop-carried
// staging pointers would otherwise compile to FLAT loads, which also count on
// the LDS wait counter: every wait for an LDS fragment would then wait for the
// in-flight prefetch as well.
__device__ __forceinline__ u32x4 ldg16(const uint16_t *p) {
  return *(const __attribute__((address_space(1))) u32x4 *)(p);
}

template <int DT> struct PipeMfma;
template <> struct PipeMfma<BF16> {
  static __device__ __forceinline__ void mma(f32x4 &c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                0, 0);
  }
  static __device__ __forceinline__ void mma0(f32x4 &c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
  }
};
template <> struct PipeMfma<F16> {
  static __device__ __forceinline__ void mma(f32x4 &c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                               0);
  }
  static __device__ __forceinline__ void mma0(f32x4 &c, u32x4 a, u32x4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                               f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
  }
};

template <int DT, int BM, int BN, int WGM, int WGN>
__global__ void __launch_bounds__(WGM * WGN * 64)
gemm_pipe_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ Bt, int M, int N, int K, long lda,
                 long ldb, long sa, long sb, long sc, EpiArgs ep) {
  constexpr int NT = WGM * WGN * 64, BK = 64;
  constexpr int WTM = BM / WGM, WTN = BN / WGN, FM = WTM / 16, FN = WTN / 16;
  constexpr int ACH = BM * 8 / NT, BCH = BN * 8 / NT;
  static_assert(ACH >= 1 && BCH >= 1 && BM * 8 % NT == 0 && BN * 8 % NT == 0 && WTM % 16 == 0 && WTN % 16 == 0,
                "tile does not fit the thread count");
  __shared__ u32x4 lds[2][(BM + BN) * 8];  // [buf][A rows | Bt rows][8 chunks], chunk-swizzled

  // ---- tile scheduling: XCD band, then group-M (same order as gemm.hip) ----
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, ntiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  constexpr int GROUP = 8;
  const int span = GROUP * tiles_n, gid = pid / span, fm = gid * GROUP, gs = min(tiles_m - fm, GROUP);
  const int tm = fm + (pid % span) % gs, tn = (pid % span) / gs;
  const int m0 = tm * BM, n0 = tn * BN;
  const int z = blockIdx.z;
  A += z * sa;
  Bt += z * sb;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave / WGN, wn = wave % WGN;
  const int li = lane & 15, lg = lane >> 4;
  // each thread stages chunk c0 (8 values) of rows r0 + RSTEP * i of A and Bt;
  // rows past M / N read the last valid row (their results are not stored).
  // Offsets are 32-bit element offsets from the slab base pointers As / Bs,
  // which advance one slab per K step (the host checks they fit).
  constexpr int RSTEP = NT / 8;
  const int c0 = tid & 7, r0 = tid >> 3;
  uint32_t aoff[ACH], boff[BCH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) aoff[i] = uint32_t(min(m0 + r0 + RSTEP * i, M - 1)) * uint32_t(lda) + c0 * 8;
#pragma unroll
  for (int i = 0; i < BCH; ++i) boff[i] = uint32_t(min(n0 + r0 + RSTEP * i, N - 1)) * uint32_t(ldb) + c0 * 8;
  const int sw = r0 * 8 + (c0 ^ (r0 & 7));  // row r0 + RSTEP * i sits at sw + RSTEP * 8 * i
  const uint16_t *As = A, *Bs = Bt;
  u32x4 ra[ACH], rb[BCH];
#define MH_PGLOAD()                                                                                \
  {                                                                                                \
    _Pragma("unroll") for (int i = 0; i < ACH; ++i) ra[i] = ldg16(As + aoff[i]);                   \
    _Pragma("unroll") for (int i = 0; i < BCH; ++i) rb[i] = ldg16(Bs + boff[i]);                   \
  }
#define MH_PSTORE(L)                                                                               \
  {                                                                                                \
    _Pragma("unroll") for (int i = 0; i < ACH; ++i)(L)[sw + RSTEP * 8 * i] = ra[i];                \
    _Pragma("unroll") for (int i = 0; i < BCH; ++i)(L)[BM * 8 + sw + RSTEP * 8 * i] = rb[i];       \
  }
  // accumulators: the first MFMA of each starts from a zero C operand (an
  // inline constant), so they are never initialised by VALU writes and keep
  // one register assignment through the K loop
  f32x4 acc[FM][FN];
  // fragments of one 32-wide K step: lane (li, lg) holds row li, chunk ks*4+lg
  u32x4 af0[FM], bf0[FN], af1[FM], bf1[FN];
#define MH_PFRAG(L, KS, AF, BF)                                                                    \
  {                                                                                                \
    const u32x4 *as_ = (L), *bs_ = (L) + BM * 8;                                                   \
    const int c = (KS) * 4 + lg;                                                                   \
    _Pragma("unroll") for (int i = 0; i < FM; ++i) {                                               \
      const int r = wm * WTM + i * 16 + li;                                                        \
      AF[i] = as_[r * 8 + (c ^ (r & 7))];                                                          \
    }                                                                                              \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) {                                               \
      const int r = wn * WTN + j * 16 + li;                                                        \
      BF[j] = bs_[r * 8 + (c ^ (r & 7))];                                                          \
    }                                                                                              \
  }
#define MH_PMMA(AF, BF)                                                                            \
  _Pragma("unroll") for (int i = 0; i < FM; ++i) _Pragma("unroll") for (int j = 0; j < FN; ++j)   \
      PipeMfma<DT>::mma(acc[i][j], BF[j], AF[i]);
#define MH_PMMA0(AF, BF)                                                                           \
  _Pragma("unroll") for (int i = 0; i < FM; ++i) _Pragma("unroll") for (int j = 0; j < FN; ++j)   \
      PipeMfma<DT>::mma0(acc[i][j], BF[j], AF[i]);
  // Instruction interleaving for the two phases of a K step (groups are
  // filled in order: MFMA, then the memory operation of that slot).
  //   phase A: each of the first NWR MFMAs is followed by one LDS store of the
  //            next slab and one global load of the slab after it, the next
  //            NRD by one fragment read of the second K half;
  //   phase B: each of the first NRD MFMAs is followed by one fragment read of
  //            the next slab's first K half.
  constexpr int NMM = FM * FN, NRD = FM + FN, NWR = ACH + BCH;
#define MH_SCHED_A()                                                                               \
  _Pragma("unroll") for (int t = 0; t < NMM; ++t) {                                                \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                             \
    if (t < NWR) {                                                                                 \
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                                           \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                           \
    } else if (t < NWR + NRD) {                                                                    \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                           \
    }                                                                                              \
  }
#define MH_SCHED_B()                                                                               \
  _Pragma("unroll") for (int t = 0; t < NMM; ++t) {                                                \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                             \
    if (t < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                \
  }

  // bf16 fast epilogue: its bias and residual quads (lane (r, g) of fragment
  // (i, j) owns row r, columns 4g..4g+3) are requested before the K loop so
  // that their memory latency is hidden behind it
  const bool fast_epi = DT == BF16 && ep.mode != EPI_CONVT && N % 4 == 0 && (!ep.resid || (ep.ldr & 3) == 0);
  // (one uniform branch per operand; rows / columns past the edge load the
  // last valid quad, whose results are not stored)
  uint2 bq[FN], rq[FM][FN];
  if (fast_epi && ep.bias) {
    const uint16_t *bias = static_cast<const uint16_t *>(ep.bias);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      bq[j] = *reinterpret_cast<const uint2 *>(bias + min(n0 + wn * WTN + j * 16 + lg * 4, N - 4));
  }
  if (fast_epi && ep.resid) {
    const uint16_t *resid = static_cast<const uint16_t *>(ep.resid);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const uint16_t *rrow = resid + long(min(m0 + wm * WTM + i * 16 + li, M - 1)) * ep.ldr;
#pragma unroll
      for (int j = 0; j < FN; ++j)
        rq[i][j] = *reinterpret_cast<const uint2 *>(rrow + min(n0 + wn * WTN + j * 16 + lg * 4, N - 4));
    }
  }

  // slab 0 covers columns [0, K0), K0 = K % 64 (or 64): chunks at or past K0
  // are zero; every later slab is whole
  const int KT = (K + BK - 1) / BK, K0 = K - (KT - 1) * BK;
  u32x4 *L0 = lds[0], *L1 = lds[1];
  {
    const bool cin = c0 * 8 < K0;
#pragma unroll
    for (int i = 0; i < ACH; ++i) ra[i] = cin ? ldg16(As + aoff[i]) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < BCH; ++i) rb[i] = cin ? ldg16(Bs + boff[i]) : u32x4{0, 0, 0, 0};
  }
  MH_PSTORE(L0);
  if (KT == 1) {
    __syncthreads();
    MH_PFRAG(L0, 0, af0, bf0);
    MH_PFRAG(L0, 1, af1, bf1);
    MH_PMMA0(af0, bf0);
    MH_PMMA(af1, bf1);
  } else {
    As += K0;
    Bs += K0;
    MH_PGLOAD();
    __syncthreads();
    MH_PFRAG(L0, 0, af0, bf0);
    // K step k: slab k in L0 with its first-half fragments in af0 / bf0, slab
    // k + 1 in the staging registers.  The loads of a step past the last slab
    // re-read the last slab (always whole, so in bounds); their data is stored
    // to the idle buffer and never read.  Step 0 is peeled: its first MFMAs
    // start the accumulators.
#define MH_PSTEP(KNEXT, MMAA)                                                                      \
  {                                                                                                \
    MH_PSTORE(L1);                                                                                 \
    if ((KNEXT) < KT) {                                                                            \
      As += BK;                                                                                    \
      Bs += BK;                                                                                    \
    }                                                                                              \
    MH_PGLOAD();                                                                                   \
    MH_PFRAG(L0, 1, af1, bf1);                                                                     \
    MMAA(af0, bf0);                                                                                \
    MH_SCHED_A();                                                                                  \
    __syncthreads();                                                                               \
    MH_PFRAG(L1, 0, af0, bf0);                                                                     \
    MH_PMMA(af1, bf1);                                                                             \
    MH_SCHED_B();                                                                                  \
    u32x4 *t = L0;                                                                                 \
    L0 = L1;                                                                                       \
    L1 = t;                                                                                        \
  }
    MH_PSTEP(2, MH_PMMA0);
    for (int k = 1; k < KT; ++k) MH_PSTEP(k + 2, MH_PMMA);
#undef MH_PSTEP
  }
#undef MH_PGLOAD
#undef MH_PSTORE
#undef MH_PFRAG
#undef MH_PMMA
#undef MH_PMMA0
#undef MH_SCHED_A
#undef MH_SCHED_B

  // ---- epilogue ----
  const long off = ep.mode == EPI_ROWMAJOR ? z * sc : 0;
  if (fast_epi) {
    // straight from the accumulators: every fragment takes the bf16 fast
    // path (bias / residual quads were loaded before the K loop)
    // destination = column part (per fragment column) + row part (per
    // fragment row): the head-split index divisions run FM + FN times, not
    // FM * FN times
    uint16_t *cbase[FN];
    long roff[FM];
    bool al8;
    if (ep.mode == EPI_HEADSPLIT) {
      // [B, T, 3E] -> q/k/v [B, H, T, hd]: row (b, t), column (which, h, dd)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = min(n0 + wn * WTN + j * 16 + lg * 4, N - 4);
        const int which = n / ep.E, e = n - which * ep.E, h = e / ep.hd, dd = e - h * ep.hd;
        uint16_t *o = static_cast<uint16_t *>(which == 0 ? ep.outs[0] : which == 1 ? ep.outs[1] : ep.outs[2]);
        cbase[j] = o + long(h) * ep.T * ep.hd + dd;
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = min(m0 + wm * WTM + i * 16 + li, M - 1);
        const int b = m / ep.T, t = m - b * ep.T;
        roff[i] = (long(b) * ep.H * ep.T + t) * ep.hd;
      }
      al8 = (ep.hd & 3) == 0 && ((uintptr_t)ep.outs[0] & 7) == 0 && ((uintptr_t)ep.outs[1] & 7) == 0 &&
            ((uintptr_t)ep.outs[2] & 7) == 0;
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j) cbase[j] = static_cast<uint16_t *>(ep.out) + off + n0 + wn * WTN + j * 16 + lg * 4;
#pragma unroll
      for (int i = 0; i < FM; ++i) roff[i] = long(m0 + wm * WTM + i * 16 + li) * ep.ldc;
      al8 = ((uintptr_t)ep.out & 7) == 0 && (ep.ldc & 3) == 0 && (off & 3) == 0;
    }
    // the epilogue kinds the engine emits run a fragment loop with the
    // chain fixed at compile time; any other (bias added before rounding,
    // unaligned destination) takes the loop with runtime branches
    // interior tiles (the common case) store every fragment unconditionally
    const bool interior = m0 + BM <= M && n0 + BN <= N;
#define MH_EPI_FIXED(BIAS, ACT, RESID)                                                              \
  _Pragma("unroll") for (int i = 0; i < FM; ++i) {                                                 \
    const int m = m0 + wm * WTM + i * 16 + li;                                                     \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) {                                               \
      const int n = n0 + wn * WTN + j * 16 + lg * 4;                                               \
      if (interior || (m < M && n < N)) {                                                          \
        float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};                     \
        *reinterpret_cast<uint2 *>(cbase[j] + roff[i]) =                                           \
            epi_fast_bf16_fixed<BIAS, ACT, RESID>(v, bq[j], rq[i][j], ep.gelu_c);                  \
      }                                                                                            \
    }                                                                                              \
  }
    const bool fixed = al8 && !(ep.bias && ep.bias_first);
    const bool hb = ep.bias != nullptr, hr = ep.resid != nullptr;
    if (fixed && !hb && ep.act == ACT_NONE && !hr) {
      MH_EPI_FIXED(false, ACT_NONE, false);
    } else if (fixed && hb && ep.act == ACT_NONE && !hr) {
      MH_EPI_FIXED(true, ACT_NONE, false);
    } else if (fixed && hb && ep.act == ACT_GELU && !hr) {
      MH_EPI_FIXED(true, ACT_GELU, false);
    } else if (fixed && hb && ep.act == ACT_RELU && !hr) {
      MH_EPI_FIXED(true, ACT_RELU, false);
    } else if (fixed && hb && ep.act == ACT_NONE && hr) {
      MH_EPI_FIXED(true, ACT_NONE, true);
    } else if (fixed && !hb && ep.act == ACT_NONE && hr) {
      MH_EPI_FIXED(false, ACT_NONE, true);
    } else {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm * WTM + i * 16 + li;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int n = n0 + wn * WTN + j * 16 + lg * 4;
          if (m < M && n < N) {
            float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            const uint2 pk = epi_fast_bf16_value(ep, v, bq[j], rq[i][j]);
            uint16_t *dst = cbase[j] + roff[i];
            if (al8) {
              *reinterpret_cast<uint2 *>(dst) = pk;
            } else {
              dst[0] = uint16_t(pk.x); dst[1] = uint16_t(pk.x >> 16); dst[2] = uint16_t(pk.y); dst[3] = uint16_t(pk.y >> 16);
            }
          }
        }
      }
    }
#undef MH_EPI_FIXED
  } else {
    // general epilogue (fp16 rounding, transposed-conv scatter, ragged N)
    // through the idle LDS
    __syncthreads();
    store_tile<DT, BM, BN, WTM, WTN, FM, FN, WGM * WGN>(acc, reinterpret_cast<float *>(&lds[0][0]), ep,
                                                       m0 + wm * WTM, n0 + wn * WTN, M, N, wave, lane, off);
  }
}

template <int DT, int BM, int BN, int WGM, int WGN>
void launch(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa, long sb,
            long sc, const EpiArgs &ep, hipStream_t st) {
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_pipe_kernel<DT, BM, BN, WGM, WGN>), dim3(tiles, 1, batch), dim3(WGM * WGN * 64), 0, st,
                     (const uint16_t *)A, (const uint16_t *)Bt, M, N, K, lda, ldb, sa, sb, sc, ep);
}

template <int DT>
hipError_t launch_dt(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
                     long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st) {
  if (tile < 0) {
    // measured on MI355X (decoder shapes, K = 768 / 3072): 128x128 when N
    // tiles evenly by 128 and there are >= 2.5 tiles per CU, 128x96 when N
    // tiles evenly by 96 (its 64x48 wave tiles fill the chip on narrow N),
    // else 128x128 / 128x64 / 64x64 by tile count
    const long t128 = long((M + 127) / 128) * ((N + 127) / 128) * batch;
    const long t64 = long((M + 127) / 128) * ((N + 63) / 64) * batch;
    if (N % 128 == 0 && t128 >= 640) tile = 0;
    else if (N % 96 == 0) tile = 3;
    else tile = (t128 >= 640 || (K >= 2048 && t128 >= 128)) ? 0 : (t64 >= 256 ? 1 : 2);
  }
  switch (tile) {
  case 0: launch<DT, 128, 128, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 1: launch<DT, 128, 64, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
  case 3: launch<DT, 128, 96, 2, 2>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, st); break;
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

hipError_t gemm_pipe(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                     long sa, long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st) {
  if (M <= 0 || N <= 0 || batch <= 0) return hipSuccess;
  if (!gemm_pipe_ok(dt, A, Bt, M, N, K, lda, ldb, sa, sb)) return hipErrorInvalidValue;
  if (dt == BF16) return launch_dt<BF16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile, st);
  return launch_dt<F16>(A, Bt, M, N, K, lda, ldb, batch, sa, sb, sc, ep, tile, st);
}

}  // namespace mh
