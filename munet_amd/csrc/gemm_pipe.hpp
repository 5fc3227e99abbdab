// Pipelined 16-bit MFMA GEMM kernels for gfx950: C[M,N] = A[M,K] * Bt[N,K]^T
// with the fused epilogue of gemm_common.hpp (the reference semantics are
// those of BackendBlasCapability::matmul and nn::Linear,
// src/core/backend.hpp:250-260, src/nn/linear.hpp:28-34).
//
// The hot path of the decoder's Linear layers (bf16/fp16, 16-byte aligned
// K-contiguous operands).  Two kernels share the tile scheduler, the LDS
// layout (128-byte K slabs, chunk c of row r at c ^ (r & 7)), the fragment
// reads, the MFMA schedule and the epilogue:
//
// gemm_pipe_kernel (register staging, any K % 8 == 0):
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
//     advance one slab per step.
//
// gemm_dma_kernel (direct-to-LDS, K % 64 == 0):
//   * slabs go from memory straight into S LDS stages with
//     global_load_lds_dwordx4 (one wave instruction fills 1 KB = 8 slab rows;
//     lane l fetches the global chunk that the swizzle places at LDS slot l),
//     so no staging registers and no LDS stores are needed: measured on
//     MI355X, the staging stores were the largest single cost of the
//     register-staged loop;
//   * the loads are issued from inline assembly, which the compiler's
//     wait-count pass does not see; the kernel waits for them itself
//     (vmcnt before each barrier, and vmcnt(0) before the epilogue and before
//     any LDS reuse).  Left to the compiler, every LDS fragment read would
//     wait for every load in flight, as it cannot tell the stages apart;
//   * step k multiplies slab k from stage k % S while slabs k + 1 .. k + S - 1
//     are in flight; phase A issues slab k + S - 1 into the stage that slab
//     k - 1 used (free since the previous barrier); steps past the last slab
//     re-load the last slab into the idle stage so that the wait counts are
//     the same on every step.
//
// Both: the epilogue runs on each accumulator fragment in registers (no LDS
// staging): lane (r, g) of a 16x16 fragment owns row r, columns 4g..4g+3; its
// bias loads (wave tiles below 128x128) and residual loads (wave tiles up to
// 64x64) are issued before the K loop.  The epilogue program is a template
// parameter (PipeKind).  Instantiated by gemm_pipe.hip (the general program,
// block tiles up to 128 rows, accumulators in VGPRs), gemm_pipe_fixed_*.hip
// (the fixed bf16 programs), gemm_pipe_wide.hip (the eight-wave tiles) and
// gemm_pipe_conv.hip (the convolutions).
#pragma once

#include "mh_common.hpp"
#include "mh_kernels.hpp"
#include "gemm_common.hpp"

namespace mh {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

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

// Output tile of this workgroup.  Workgroups are dealt round-robin to the 8
// XCDs (pid & 7), each with its own L2, so the tile index is first remapped
// to give each XCD a contiguous eighth of an enumeration of the tile grid.
// gn = 0: the enumeration walks groups of GROUP tile rows across all
// columns, so an XCD holds a band of A rows and about half of W (A is read
// about twice, W about four times; best when A is the larger operand).
// gn > 0: it walks groups of gn tile columns, row by row across the group,
// so an XCD holds about 1/8 of W and A is re-read once per group (best when W
// is as large as A or larger: the weights arrive cold from HBM in a forward).
template <int BM, int BN>
__device__ __forceinline__ void pipe_tile(int M, int N, int gn, int &m0, int &n0) {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, ntiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  constexpr int GROUP = 8;
  if (gn > 0 && (ntiles & 7) == 0) {
    const int t = (pid & 7) * (ntiles >> 3) + (pid >> 3), span = gn * tiles_m;
    const int g = t / span, r = t - g * span, w = min(gn, tiles_n - g * gn);
    m0 = (r / w) * BM;
    n0 = (g * gn + r % w) * BN;
    return;
  }
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int span = GROUP * tiles_n, gid = pid / span, fm = gid * GROUP, gs = min(tiles_m - fm, GROUP);
  m0 = (fm + (pid % span) % gs) * BM;
  n0 = ((pid % span) / gs) * BN;
}

// Wave-level geometry of a BM x BN block tile on WGM x WGN waves and the MFMA
// fragment reads: fragments of one 32-wide K half KS of the slab in L; lane
// (li, lg) holds row li, chunk KS*4 + lg of each 16-row fragment.
template <int BM, int BN, int WGM, int WGN> struct PipeGeom {
  static constexpr int NW = WGM * WGN, NT = NW * 64;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN, FM = WTM / 16, FN = WTN / 16;
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile");
  int wm, wn, li, lg;
  __device__ __forceinline__ PipeGeom(int wave, int lane)
      : wm(wave / WGN), wn(wave % WGN), li(lane & 15), lg(lane >> 4) {}
  template <int KS>
  __device__ __forceinline__ void frags(const u32x4 *L, u32x4 (&af)[FM], u32x4 (&bf)[FN]) const {
    const u32x4 *as = L, *bs = L + BM * 8;
    const int c = KS * 4 + lg;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = wm * WTM + i * 16 + li;
      af[i] = as[r * 8 + (c ^ (r & 7))];
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int r = wn * WTN + j * 16 + li;
      bf[j] = bs[r * 8 + (c ^ (r & 7))];
    }
  }
};

// Epilogue programs.  PK_GENERAL serves every EpiArgs (a fragment loop with
// the rounding chain chosen at run time, or the LDS-staged store_tile for
// fp16, transposed-conv scatter and ragged N).  The others are the
// combinations the engine emits, each one fragment loop fixed at compile
// time, so a kernel carries only its own epilogue (bf16, 8-byte aligned
// destination, bias added after the matmul rounding; the host checks).  One
// epilogue per kernel keeps the code small: with every variant inlined the
// kernels grew to 30k instructions, and kernels replayed in a graph refetch
// their code each launch.
enum PipeKind : int {
  PK_GENERAL = 0,
  PK_PLAIN,          // round(acc)
  PK_BIAS,           // + bias
  PK_BIAS_GELU,      // + bias, GELU
  PK_BIAS_RESID,     // + bias, + residual
  PK_LN_BIAS,        // folded LayerNorm consumer, + bias
  PK_LN_BIAS_GELU,   // folded LayerNorm consumer, + bias, GELU
  PK_BIAS_RESID_ST,  // + bias, + residual, writes LayerNorm partials
  PK_BIAS_NT,        // + bias, non-temporal stores (an output no kernel reads)
  PK_COUNT
};
template <int EK> struct PipeKindT {
  static constexpr bool FIXED = EK != PK_GENERAL;
  static constexpr bool LN = EK == PK_LN_BIAS || EK == PK_LN_BIAS_GELU;
  static constexpr bool ST = EK == PK_BIAS_RESID_ST;
  static constexpr bool BIAS = FIXED && EK != PK_PLAIN;
  static constexpr int ACT = (EK == PK_BIAS_GELU || EK == PK_LN_BIAS_GELU) ? ACT_GELU : ACT_NONE;
  static constexpr bool RESID = EK == PK_BIAS_RESID || EK == PK_BIAS_RESID_ST;
  static constexpr bool NT = EK == PK_BIAS_NT;
};

// The fused epilogue of a wave's accumulator tile.  bf16 fast path: lane
// (r, g) of fragment (i, j) owns row r, columns 4g..4g+3.  Where they fit
// beside the staging and fragment registers, its bias quads (wave tiles below
// 128x128) and residual quads (wave tiles up to 64x64) are requested before
// the K loop (prefetch()) so that their memory latency is hidden behind it;
// larger wave tiles load them in store().  One uniform branch per operand;
// rows / columns past the edge load the last valid quad, whose results are
// not stored.  Other cases (fp16 rounding, transposed-conv scatter, ragged
// N) go through the general LDS-staged store_tile.
template <int DT, int BM, int BN, int WGM, int WGN, int EK> struct PipeEpi {
  typedef PipeGeom<BM, BN, WGM, WGN> G;
  typedef PipeKindT<EK> KT_;
  static constexpr int FM = G::FM, FN = G::FN, WTM = G::WTM, WTN = G::WTN;
  static constexpr bool PRE_B = FM * FN < 64, PRE_R = FM * FN <= 16;
  static constexpr int RQM = PRE_R ? FM : 1, RQN = PRE_R ? FN : 1;
  // (the epilogue arguments are passed to every method rather than held by
  // reference: a reference to the by-value kernel argument would make the
  // compiler copy it to scratch)
  const G g;
  const int M, N, m0, n0;
  const bool fast;
  uint2 bq[FN], rq[RQM][RQN];

  __device__ __forceinline__ PipeEpi(const EpiArgs &ep, const G &g_, int M_, int N_, int m0_, int n0_)
      : g(g_), M(M_), N(N_), m0(m0_), n0(n0_),
        fast(KT_::FIXED || ((DT == BF16 || DT == F16) && N_ % 4 == 0 && (!ep.resid || (ep.ldr & 3) == 0) &&
                            (ep.mode != EPI_CONVT || (ep.convt_oc % 4 == 0 && !ep.resid)))) {}

  __device__ __forceinline__ uint2 bload(const EpiArgs &ep, int j) const {
    const uint16_t *bias = static_cast<const uint16_t *>(ep.bias);
    int n = min(n0 + g.wn * WTN + j * 16 + g.lg * 4, N - 4);
    if (!KT_::FIXED && ep.mode == EPI_CONVT) n %= ep.convt_oc;  // column (tap, oc): the bias of oc
    return *reinterpret_cast<const uint2 *>(bias + n);
  }
  __device__ __forceinline__ uint2 rload(const EpiArgs &ep, int i, int j) const {
    const uint16_t *resid = static_cast<const uint16_t *>(ep.resid);
    return *reinterpret_cast<const uint2 *>(resid + long(min(m0 + g.wm * WTM + i * 16 + g.li, M - 1)) * ep.ldr +
                                           min(n0 + g.wn * WTN + j * 16 + g.lg * 4, N - 4));
  }

  __device__ __forceinline__ bool has_bias(const EpiArgs &ep) const { return KT_::FIXED ? KT_::BIAS : ep.bias != nullptr; }
  __device__ __forceinline__ bool has_resid(const EpiArgs &ep) const {
    return KT_::FIXED ? KT_::RESID : ep.resid != nullptr;
  }
  // vector loads prefetch() issues for a fixed program (one 8-byte load per
  // bias fragment column and per residual fragment)
  static constexpr int NPRE = (PRE_B && KT_::BIAS ? FN : 0) + (PRE_R && KT_::RESID ? FM * FN : 0);
  __device__ __forceinline__ void prefetch(const EpiArgs &ep) {
    if (PRE_B && fast && has_bias(ep)) {
#pragma unroll
      for (int j = 0; j < FN; ++j) bq[j] = bload(ep, j);
    }
    if (PRE_R && fast && has_resid(ep)) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) rq[i][j] = rload(ep, i, j);
    }
  }

  // Folded LayerNorm, consumer prologue.  ln_issue() requests this tile's
  // inputs before the kernel's first slab: NT / BM threads per row each load
  // a contiguous share (up to LNCH) of the row's partials into registers,
  // two partials per 16-byte load where the row length allows, and threads
  // t < BN load column t's folded-weight sum and beta W.  ln_finish() runs
  // once the first slab has landed (the same memory round trip): it combines
  // the shares with Chan's parallel-variance formula, then across adjacent
  // lanes, and writes (mean, rstd) per row and the column terms to LDS; the
  // K loop's barriers make them visible to the epilogue.
  // (tiles of fewer rows than NT / 4, which never fold a LayerNorm, size the
  // slots as for 4 threads per row; ln_issue / ln_finish reject them)
  static constexpr int TPR = G::NT / BM < 4 ? G::NT / BM : 4, LNCH = 32, CH = 4 / TPR;
  static_assert(TPR == 1 || TPR == 2 || TPR == 4, "threads per row");
  // A row's partials are split into 4 chunks of `chunk` (even) partials; each
  // chunk is combined in order, then the chunks pairwise, (0 1) (2 3) and
  // then the two pairs, the lower one first.  A thread owns CH consecutive
  // chunks, so every tile combines in the same order whatever its threads
  // per row, and gives the same bits.
  static __device__ __forceinline__ int ln_chunk(int P) { return ((P + 3) / 4 + 1) & ~1; }
  // (explicit fma / mul / add: HIP contracts a * b + c into an fma where the
  // optimiser chooses, which differs between kernel instantiations; these
  // statistics must round the same in every tile)
  static __device__ __forceinline__ void chan_pair(float &n, float &mean, float &m2, float on, float om, float o2) {
    const float nn = __fadd_rn(n, on), d = __fsub_rn(om, mean);
    if (nn > 0.f) {
      const float f = __fdiv_rn(on, nn);
      mean = __fmaf_rn(d, f, mean);
      m2 = __fadd_rn(m2, __fadd_rn(o2, __fmul_rn(__fmul_rn(d, d), __fmul_rn(n, f))));
    }
    n = nn;
  }
  struct LnIn {
    float4 part[LNCH / 2];  // (mean, M2) pairs
    float cs, bw;
  };
  // (loads are unconditional, at indices clamped into the row; ln_finish
  // counts only the share's own partials)
  // chunk c of this thread lands at in.part[c * LPC / 2 ..] (LPC partials
  // per chunk slot), so every index below is a compile-time constant
  static constexpr int LPC = LNCH / CH;
  __device__ __forceinline__ void ln_issue(const EpiArgs &ep, LnIn &in, int tid) const {
    static_assert(G::NT / BM <= 4, "a folded LayerNorm needs at most 4 threads per tile row");
    // a chunk holds up to ln_chunk(64) = 16 partials (the host admits 64 per
    // row): every tile that folds a LayerNorm needs room for all of them
    static_assert(LPC >= 16, "LayerNorm chunk slot smaller than the largest chunk");
    const int r = tid / TPR, q = tid % TPR, P = ep.ln_parts, chunk = ln_chunk(P);
    const long row = min(m0 + r, M - 1);
    if ((P & 1) == 0) {  // rows and chunks start on 16-byte boundaries: two partials per load
      const float4 *p4 = reinterpret_cast<const float4 *>(ep.ln_stats) + row * (P / 2);
      const int last = P / 2 - 1;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int k0 = (q * CH + c) * chunk;
#pragma unroll
        for (int i = 0; i < LPC / 2; ++i)
          if (2 * i < chunk) in.part[c * LPC / 2 + i] = p4[min(k0 / 2 + i, last)];
      }
    } else {
      const float2 *p = reinterpret_cast<const float2 *>(ep.ln_stats) + row * P;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int k0 = (q * CH + c) * chunk;
#pragma unroll
        for (int i = 0; i < LPC / 2; ++i) {
          if (2 * i < chunk) {
            const float2 a = p[min(k0 + 2 * i, P - 1)], b = p[min(k0 + 2 * i + 1, P - 1)];
            in.part[c * LPC / 2 + i] = make_float4(a.x, a.y, b.x, b.y);
          }
        }
      }
    }
    const int c = min(n0 + min(tid, BN - 1), N - 1);
    in.cs = ep.ln_cs[c];
    in.bw = ep.ln_bw[c];
  }
  // Chan's in-order combine of one chunk's partials (slots i < NI of chunk
  // slot c; with CHECK only those below `chunk`)
  template <int NI, bool CHECK>
  static __device__ __forceinline__ void chunk_stats(const LnIn &in, int c, int chunk, int k0, int k1, float &mean,
                                                     float &m2, float &m2x) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int j = c * LPC + i;  // index into this thread's loaded partials
      if ((!CHECK || i < chunk) && k0 + i < k1) {
        const float pm = j & 1 ? in.part[j / 2].z : in.part[j / 2].x;
        const float p2 = j & 1 ? in.part[j / 2].w : in.part[j / 2].y;
        const float d = __fsub_rn(pm, mean);
        mean = __fmaf_rn(d, 1.0f / float(i + 1), mean);
        m2 = __fadd_rn(m2, p2);
        m2x = __fmaf_rn(__fmul_rn(d, d), float(i) / float(i + 1), m2x);
      }
    }
  }
  __device__ __forceinline__ void ln_finish(const EpiArgs &ep, const LnIn &in, float2 *lnrow, float *lncs,
                                            float *lnbw, int tid) const {
    const int r = tid / TPR, q = tid % TPR, P = ep.ln_parts, chunk = ln_chunk(P);
    // every partial covers w columns, so after i partials of a chunk n = i w
    // and Chan's update weights are the constants 1 / (i + 1) and i / (i + 1)
    const float w = float(ep.ln_cols);
    float cn[CH], cm[CH], c2[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k0 = (q * CH + c) * chunk, k1 = min(k0 + chunk, P);
      float mean = 0.f, m2 = 0.f, m2x = 0.f;  // m2x: the between-partial term / w
      // the chunk length is the same for every lane: the usual lengths (the
      // decoder's 8 and 16 partials per row) take loops of exactly that many
      // slots; the rest run all LPC slots predicated
      if (chunk == 2)
        chunk_stats<2, false>(in, c, 2, k0, k1, mean, m2, m2x);
      else if (chunk == 4)
        chunk_stats<4, false>(in, c, 4, k0, k1, mean, m2, m2x);
      else
        chunk_stats<LPC, true>(in, c, chunk, k0, k1, mean, m2, m2x);
      cm[c] = mean;
      c2[c] = __fmaf_rn(m2x, w, m2);
      cn[c] = float(max(k1 - k0, 0)) * w;
    }
    // chunks of this thread: (0 1), (2 3), then the pairs
#pragma unroll
    for (int o = 1; o < CH; o <<= 1)
#pragma unroll
      for (int c = 0; c < CH; c += 2 * o) chan_pair(cn[c], cm[c], c2[c], cn[c + o], cm[c + o], c2[c + o]);
    float n = cn[0], mean = cm[0], m2 = c2[0];
    // then across the row's threads (the lower lane's values first)
#pragma unroll
    for (int o = 1; o < TPR; o <<= 1) {
      const float on = __shfl_xor(n, o), om = __shfl_xor(mean, o), o2 = __shfl_xor(m2, o);
      if (q & o) {
        float tn = on, tm = om, t2 = o2;
        chan_pair(tn, tm, t2, n, mean, m2);
        n = tn, mean = tm, m2 = t2;
      } else {
        chan_pair(n, mean, m2, on, om, o2);
      }
    }
    if (q == 0) lnrow[r] = make_float2(mean, __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(m2, n), ep.ln_eps))));
    if (tid < BN) {
      lncs[tid] = in.cs;
      lnbw[tid] = in.bw;
    }
  }

  // Producer side: partials of stats_cols columns (whole groups of fragment
  // columns inside a wave tile).  Each lane keeps the 4 rounded values it
  // owns in every fragment column of the group (row li, columns 4 lg ..
  // 4 lg + 3); when the group is complete, the row's sum and then its sum of
  // squared deviations are reduced across the 4 lanes that share the row
  // (lanes li, li+16, li+32, li+48) and lane group 0 stores (mean, M2).
  struct StatAcc {
    float y[FN][4];
  };
  __device__ __forceinline__ void stats_add(const EpiArgs &ep, StatAcc &a, uint2 pk, int m, int j) const {
    a.y[j][0] = lo_bf16(pk.x);
    a.y[j][1] = hi_bf16(pk.x);
    a.y[j][2] = lo_bf16(pk.y);
    a.y[j][3] = hi_bf16(pk.y);
    const int G16 = ep.stats_cols / 16;  // fragment columns per group
    if ((j + 1) % G16 == 0) {
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < FN; ++t)
        if (t <= j && t > j - G16) s += (a.y[t][0] + a.y[t][1]) + (a.y[t][2] + a.y[t][3]);
      s = xor32_add(xor16_add(s));
      const float mu = s / float(ep.stats_cols);
      float q = 0.f;
#pragma unroll
      for (int t = 0; t < FN; ++t)
        if (t <= j && t > j - G16)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float dv = __fsub_rn(a.y[t][e], mu);
            q = __fmaf_rn(dv, dv, q);  // explicit: the same rounding in every tile
          }
      q = xor32_add(xor16_add(q));
      const int g0 = n0 + g.wn * WTN + (j + 1) * 16 - ep.stats_cols;  // first column of the group
      if (g.lg == 0 && m < M && g0 < N)
        *reinterpret_cast<float2 *>(ep.stats_out + 2 * (long(m) * (N / ep.stats_cols) + g0 / ep.stats_cols)) =
            make_float2(mu, q);
    }
  }

  // Non-temporal output (an output no kernel reads, such as the logits) in
  // whole lines: each wave rounds its tile into LDS as rows of WTN values and
  // writes the rows back with 16-byte non-temporal stores, LPR lanes per row,
  // so every store instruction covers whole 128-byte lines.  Per-fragment
  // 8-byte non-temporal stores write 32-byte pieces of lines that bypass the
  // cache's write combining: measured on the vocabulary head, the memory side
  // then wrote 2.25 times the output's bytes.  Interior tiles of an aligned
  // row-major output only (the caller checks).
  static constexpr int NT_LPR = WTN * 2 / 16;  // lanes per staged row
  static constexpr int NT_RB = WTN * 2 + 16;   // bytes per staged row (16-byte pad against bank conflicts)
  // rows of its tile a wave stages at a time: all, or a half / quarter when
  // the waves' tiles do not fit the K loop's LDS (2 stages at least)
  static constexpr int NT_PASSES = WTM * NT_RB * G::NW <= 2 * (BM + BN) * 128       ? 1
                                   : (WTM / 2) * NT_RB * G::NW <= 2 * (BM + BN) * 128 ? 2
                                                                                     : 4;
  static constexpr bool NT_ROWS = WTN % 8 == 0 && NT_LPR <= 64 && 64 % NT_LPR == 0 && FM % NT_PASSES == 0 &&
                                  (WTM / NT_PASSES) * NT_RB * G::NW <= 2 * (BM + BN) * 128;
  __device__ __forceinline__ void store_nt_rows(const EpiArgs &ep, f32x4 (&acc)[FM][FN], long off, u32x4 *lds,
                                                int wave, int lane) {
    constexpr int RPI = 64 / NT_LPR;  // rows per store instruction
    constexpr int FMP = FM / NT_PASSES, RP = WTM / NT_PASSES;
    char *stage = reinterpret_cast<char *>(lds) + wave * RP * NT_RB;
    __syncthreads();  // every wave has read its last fragments from the K loop's LDS
    const int rr = lane / NT_LPR, cc = lane % NT_LPR;
    uint16_t *base = static_cast<uint16_t *>(ep.out) + off + long(m0 + g.wm * WTM) * ep.ldc + n0 + g.wn * WTN + cc * 8;
#pragma unroll
    for (int p = 0; p < NT_PASSES; ++p) {
#pragma unroll
      for (int i = 0; i < FMP; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          float v[4] = {acc[p * FMP + i][j][0], acc[p * FMP + i][j][1], acc[p * FMP + i][j][2],
                        acc[p * FMP + i][j][3]};
          const uint2 pk = epi_fast_fixed<DT, KT_::BIAS, ACT_NONE, false>(v, bq[j], make_uint2(0, 0), ep.gelu_c);
          *reinterpret_cast<uint2 *>(stage + (i * 16 + g.li) * NT_RB + (j * 16 + g.lg * 4) * 2) = pk;
        }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int r = rr; r < RP; r += RPI) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + r * NT_RB + cc * 16);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(base + long(p * RP + r) * ep.ldc));
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // the rows are read back before the next pass rewrites them
      __builtin_amdgcn_wave_barrier();
    }
  }

  // Whole-line stores of the head-split q/k/v for the fixed programs on
  // interior tiles: the waves round their fragments into LDS as the block
  // tile's rows (BN values and a 16-byte pad per row), then every thread
  // copies 16-byte chunks out with consecutive lanes on consecutive chunks of
  // a row, so each store instruction writes whole 128-byte lines (a head
  // width that is a multiple of 8: a chunk never straddles two heads).
  // Measured on the decoder's q/k/v product: 22.7 -> 21.7 us alone.  The
  // same path for row-major outputs was 0.3-0.8 us slower on the layer
  // GEMMs (their store cost is the write bandwidth, not the 32-byte pieces
  // of the per-fragment stores), so those keep the fragment stores.
  static constexpr int LN_RB = BN * 2 + 16;
  static constexpr bool LINES = BN % 8 == 0 && BN / 8 <= G::NT && BM * LN_RB <= 2 * (BM + BN) * 128;
  __device__ __forceinline__ bool lines_ok(const EpiArgs &ep, long) const {
    return ep.mode == EPI_HEADSPLIT && (ep.hd & 7) == 0 &&
           (((uintptr_t)ep.outs[0] | (uintptr_t)ep.outs[1] | (uintptr_t)ep.outs[2]) & 15) == 0;
  }
  __device__ __forceinline__ void store_lines(const EpiArgs &ep, f32x4 (&acc)[FM][FN], u32x4 *lds, int tid,
                                              const float2 *lnrow, const float *lncs, const float *lnbw) {
    const int wm = g.wm, wn = g.wn, li = g.li, lg = g.lg;
    char *stage = reinterpret_cast<char *>(lds);
    __syncthreads();  // every wave has read its last fragments from the K loop's LDS
    float4 lcs[FN], lbw[FN];
    if constexpr (KT_::LN) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        lcs[j] = *reinterpret_cast<const float4 *>(lncs + wn * WTN + j * 16 + lg * 4);
        lbw[j] = *reinterpret_cast<const float4 *>(lnbw + wn * WTN + j * 16 + lg * 4);
      }
    }
#define RQL(I, J) (!has_resid(ep) ? make_uint2(0, 0) : PRE_R ? rq[(I) % RQM][(J) % RQN] : rload(ep, I, J))
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = wm * WTM + i * 16 + li;
      float2 rs = make_float2(0.f, 0.f);
      if constexpr (KT_::LN) rs = lnrow[r];
      StatAcc sa;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        if constexpr (KT_::LN) {  // explicit fmas: the same rounding in every tile
          v[0] = __fmaf_rn(rs.y, __fmaf_rn(-rs.x, lcs[j].x, v[0]), lbw[j].x);
          v[1] = __fmaf_rn(rs.y, __fmaf_rn(-rs.x, lcs[j].y, v[1]), lbw[j].y);
          v[2] = __fmaf_rn(rs.y, __fmaf_rn(-rs.x, lcs[j].z, v[2]), lbw[j].z);
          v[3] = __fmaf_rn(rs.y, __fmaf_rn(-rs.x, lcs[j].w, v[3]), lbw[j].w);
        }
        const uint2 pk = epi_fast_fixed<DT, KT_::BIAS, KT_::ACT, KT_::RESID>(v, bq[j], RQL(i, j), ep.gelu_c);
        *reinterpret_cast<uint2 *>(stage + r * LN_RB + (wn * WTN + j * 16 + lg * 4) * 2) = pk;
        if constexpr (KT_::ST) stats_add(ep, sa, pk, m0 + r, j);
      }
    }
#undef RQL
    __syncthreads();
    constexpr int CPR = BN / 8, RPP = G::NT / CPR;  // chunks per row, rows per pass
    const int cc = tid % CPR, rr = tid / CPR;
    if (rr >= RPP) return;
    const int n = n0 + cc * 8;
    const char *src = stage + rr * LN_RB + cc * 16;
    {
      // column n = which E + h hd + dd (E = H hd); row m = b T + t
      const int hq = n / ep.hd, dd = n - hq * ep.hd, which = hq / ep.H, h = hq - which * ep.H;
      const uintptr_t o = which == 0 ? reinterpret_cast<uintptr_t>(ep.outs[0])
                          : which == 1 ? reinterpret_cast<uintptr_t>(ep.outs[1])
                                       : reinterpret_cast<uintptr_t>(ep.outs[2]);
      uint16_t *colp = reinterpret_cast<uint16_t *>(o) + long(h) * ep.T * ep.hd + dd;
      int b = (m0 + rr) / ep.T, t = m0 + rr - b * ep.T;
#pragma unroll
      for (int k = 0; k < (BM + RPP - 1) / RPP; ++k) {
        if (rr + k * RPP < BM)
          *reinterpret_cast<u32x4 *>(colp + (long(b) * ep.H * ep.T + t) * ep.hd) =
              *reinterpret_cast<const u32x4 *>(src + k * RPP * LN_RB);
        t += RPP;
        while (t >= ep.T) t -= ep.T, ++b;
      }
    }
  }

  // lds: the kernel's LDS (idle by now), at least 2 * (BM + BN) * 128 bytes;
  // lnrow, lncs, lnbw: the folded LayerNorm's row and column terms
  // (ln_finish)
  __device__ __forceinline__ void store(const EpiArgs &ep, f32x4 (&acc)[FM][FN], long off, u32x4 *lds, int wave,
                                        int lane, const float2 *lnrow, const float *lncs, const float *lnbw) {
    const int wm = g.wm, wn = g.wn, li = g.li, lg = g.lg;
    if (!fast) {
      __syncthreads();
      store_tile<DT, BM, BN, WTM, WTN, FM, FN, G::NW>(acc, reinterpret_cast<float *>(lds), ep, m0 + wm * WTM,
                                                      n0 + wn * WTN, M, N, wave, lane, off);
      return;
    }
    if (!PRE_B && has_bias(ep)) {
#pragma unroll
      for (int j = 0; j < FN; ++j) bq[j] = bload(ep, j);
    }
    if constexpr (KT_::FIXED && !KT_::NT && LINES) {
      if (m0 + BM <= M && n0 + BN <= N && lines_ok(ep, off)) {
        store_lines(ep, acc, lds, wave * 64 + lane, lnrow, lncs, lnbw);
        return;
      }
    }
    // destination = column part (per fragment column) + row part (per
    // fragment row): the head-split index divisions run FM + FN times, not
    // FM * FN times
    uint16_t *cbase[FN];
    long roff[FM];
    bool al8;
    if (ep.mode == EPI_HEADSPLIT) {
      // [B, T, 3E] -> q/k/v [B, H, T, hd]: row (b, t), column (which, h, dd).
      // The three destinations are selected as integer values: a select
      // between the addresses of ep.outs[i] would need the arguments in
      // private memory.
      const uintptr_t o0 = reinterpret_cast<uintptr_t>(ep.outs[0]), o1 = reinterpret_cast<uintptr_t>(ep.outs[1]),
                      o2 = reinterpret_cast<uintptr_t>(ep.outs[2]);
      const long thd = long(ep.T) * ep.hd;
      if (ep.hd >= 16) {
        // one division for the lane's first column, then 16-column steps
        // (hd >= 16: a step crosses at most one head boundary); column
        // n = which E + h hd + dd with E = H hd.  Columns past N keep
        // counting: their stores are masked.
        const int hq = (n0 + wn * WTN + lg * 4) / ep.hd, which = hq / ep.H, h0 = hq - which * ep.H;
        int dd = n0 + wn * WTN + lg * 4 - hq * ep.hd, hleft = ep.H - h0;  // heads left in this output
        // p: byte address of the column in the current output; next: the
        // following output's base
        uintptr_t p = (which == 0 ? o0 : which == 1 ? o1 : o2) + 2 * (h0 * thd + dd);
        uintptr_t next = which == 0 ? o1 : o2;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          cbase[j] = reinterpret_cast<uint16_t *>(p);
          dd += 16;
          p += 32;
          if (dd >= ep.hd) {  // next head: skip the rest of this head's T rows
            dd -= ep.hd;
            p += 2 * (thd - ep.hd);
            if (--hleft == 0) hleft = ep.H, p = next + 2 * dd, next = o2;
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int n = min(n0 + wn * WTN + j * 16 + lg * 4, N - 4);
          const int which = n / ep.E, e = n - which * ep.E, h = e / ep.hd, dd = e - h * ep.hd;
          const uintptr_t o = which == 0 ? o0 : which == 1 ? o1 : o2;
          cbase[j] = reinterpret_cast<uint16_t *>(o) + h * thd + dd;
        }
      }
      if (ep.T >= 16) {
        // rows m = b T + t, in 16-row steps from the lane's first
        int b = (m0 + wm * WTM + li) / ep.T, t = m0 + wm * WTM + li - b * ep.T;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          roff[i] = (long(b) * ep.H * ep.T + t) * ep.hd;
          t += 16;
          if (t >= ep.T) t -= ep.T, ++b;
        }
      } else {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int m = min(m0 + wm * WTM + i * 16 + li, M - 1);
          const int b = m / ep.T, t = m - b * ep.T;
          roff[i] = (long(b) * ep.H * ep.T + t) * ep.hd;
        }
      }
      al8 = (ep.hd & 3) == 0 && ((uintptr_t)ep.outs[0] & 7) == 0 && ((uintptr_t)ep.outs[1] & 7) == 0 &&
            ((uintptr_t)ep.outs[2] & 7) == 0;
    } else if (!KT_::FIXED && ep.mode == EPI_CONVT) {
      // transposed convolution: row m = input pixel (b, ih, iw), column n =
      // (kh k + kw) oC + oc lands on output pixel (b, ih k + kh, iw k + kw),
      // channel oc; the output offset splits into a row part and a column part
      const int k = ep.convt_k, oW = ep.convt_iw * k;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = min(n0 + wn * WTN + j * 16 + lg * 4, N - 4);
        const int oc = n % ep.convt_oc, ph = n / ep.convt_oc, kh = ph / k, kw = ph - kh * k;
        cbase[j] = static_cast<uint16_t *>(ep.out) + (long(kh) * oW + kw) * ep.ldc + oc;
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = min(m0 + wm * WTM + i * 16 + li, M - 1);
        const int iw = m % ep.convt_iw, rest = m / ep.convt_iw, ih = rest % ep.convt_ih, b = rest / ep.convt_ih;
        roff[i] = ((long(b) * ep.convt_ih + ih) * k * oW + long(iw) * k) * ep.ldc;
      }
      al8 = ((uintptr_t)ep.out & 7) == 0 && (ep.ldc & 3) == 0;
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j) cbase[j] = static_cast<uint16_t *>(ep.out) + off + n0 + wn * WTN + j * 16 + lg * 4;
#pragma unroll
      for (int i = 0; i < FM; ++i) roff[i] = long(m0 + wm * WTM + i * 16 + li) * ep.ldc;
      al8 = ((uintptr_t)ep.out & 7) == 0 && (ep.ldc & 3) == 0 && (off & 3) == 0;
    }
    // Interior tiles (the common case) store every fragment unconditionally.
    const bool interior = m0 + BM <= M && n0 + BN <= N;
    if constexpr (KT_::NT && NT_ROWS) {
      if (interior && ep.mode == EPI_ROWMAJOR && (ep.ldc & 7) == 0 && (off & 7) == 0 &&
          ((uintptr_t)ep.out & 15) == 0) {
        store_nt_rows(ep, acc, off, lds, wave, lane);
        return;
      }
    }
#define RQ(I, J) (!has_resid(ep) ? make_uint2(0, 0) : PRE_R ? rq[(I) % RQM][(J) % RQN] : rload(ep, I, J))
    if constexpr (KT_::FIXED) {
      // folded LayerNorm: per-column terms (column sums of gamma (.) W,
      // beta W) from LDS (ln_finish)
      float4 lcs[FN], lbw[FN];
      if constexpr (KT_::LN) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          lcs[j] = *reinterpret_cast<const float4 *>(lncs + wn * WTN + j * 16 + lg * 4);
          lbw[j] = *reinterpret_cast<const float4 *>(lnbw + wn * WTN + j * 16 + lg * 4);
        }
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm * WTM + i * 16 + li;
        float2 rs = make_float2(0.f, 0.f);
        if constexpr (KT_::LN) rs = lnrow[wm * WTM + i * 16 + li];
        StatAcc sa;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int n = n0 + wn * WTN + j * 16 + lg * 4;
          float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
          if constexpr (KT_::LN) {  // explicit fmas: the same rounding in every tile
            v[0] = __fmaf_rn(rs.y, __fmaf_rn(-rs.x, lcs[j].x, v[0]), lbw[j].x);
            v[1] = __fmaf_rn(rs.y, __fmaf_rn(-rs.x, lcs[j].y, v[1]), lbw[j].y);
            v[2] = __fmaf_rn(rs.y, __fmaf_rn(-rs.x, lcs[j].z, v[2]), lbw[j].z);
            v[3] = __fmaf_rn(rs.y, __fmaf_rn(-rs.x, lcs[j].w, v[3]), lbw[j].w);
          }
          const uint2 pk = epi_fast_fixed<DT, KT_::BIAS, KT_::ACT, KT_::RESID>(v, bq[j], RQ(i, j), ep.gelu_c);
          if (interior || (m < M && n < N)) {
            if constexpr (KT_::NT)
              __builtin_nontemporal_store((uint64_t(pk.y) << 32) | pk.x, reinterpret_cast<uint64_t *>(cbase[j] + roff[i]));
            else
              *reinterpret_cast<uint2 *>(cbase[j] + roff[i]) = pk;
          }
          if constexpr (KT_::ST) stats_add(ep, sa, pk, m, j);
        }
      }
    } else {
      // any other chain (bias added before rounding, unaligned destination)
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm * WTM + i * 16 + li;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int n = n0 + wn * WTN + j * 16 + lg * 4;
          if (m < M && n < N) {
            float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            const uint2 pk = epi_fast_value<DT>(ep, v, bq[j], RQ(i, j));
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
#undef RQ
  }
};

// MFMAs of one 32-wide K half over the wave tile (first use: zero C operand,
// so accumulators are never initialised by VALU writes and keep one register
// assignment through the K loop)
#define MH_PMMA(AF, BF)                                                                            \
  _Pragma("unroll") for (int i = 0; i < FM; ++i) _Pragma("unroll") for (int j = 0; j < FN; ++j)   \
      PipeMfma<DT>::mma(acc[i][j], BF[j], AF[i]);
#define MH_PMMA0(AF, BF)                                                                           \
  _Pragma("unroll") for (int i = 0; i < FM; ++i) _Pragma("unroll") for (int j = 0; j < FN; ++j)   \
      PipeMfma<DT>::mma0(acc[i][j], BF[j], AF[i]);

// CONV: implicit-GEMM convolution (M = output pixels, N = oC, K = kH*kW*iC)
// on an NHWC activation A with OHWI weights Bt, iC % 64 == 0, so every
// 64-wide K slab is one filter tap (kh, kw) and 64 consecutive channels.
// Each thread keeps, per A row, the byte offset of the row's tap (0, 0)
// chunk and a bit mask of its taps that fall inside the image; a slab adds
// the tap's offset (a scalar) and loads through a buffer resource, taps in
// the padding reading an offset past the resource's end, which the hardware
// returns as zeros.
template <int DT, int BM, int BN, int WGM, int WGN, int EK, bool CONV = false>
__global__ void __launch_bounds__(WGM * WGN * 64)
gemm_pipe_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ Bt, int M, int N, int K, long lda,
                 long ldb, long sa, long sb, long sc, EpiArgs ep, ConvArgs cv) {
  typedef PipeGeom<BM, BN, WGM, WGN> G;
  constexpr int NT = G::NT, BK = 64, FM = G::FM, FN = G::FN;
  constexpr int ACH = BM * 8 / NT, BCH = BN * 8 / NT;
  static_assert(ACH >= 1 && BCH >= 1 && BM * 8 % NT == 0 && BN * 8 % NT == 0, "tile does not fit the thread count");
  __shared__ u32x4 lds[2][(BM + BN) * 8];  // [buf][A rows | Bt rows][8 chunks], chunk-swizzled
  __shared__ float2 lnrow[BM];              // folded LayerNorm: row (mean, rstd)
  __shared__ __attribute__((aligned(16))) float lncs[BN], lnbw[BN];  // and column terms

  int m0, n0;
  pipe_tile<BM, BN>(M, N, ep.xcd_gn, m0, n0);
  const int z = blockIdx.z;
  A += z * sa;
  Bt += z * sb;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const G g(wave, lane);
  // each thread stages chunk c0 (8 values) of rows r0 + RSTEP * i of A and Bt;
  // rows past M / N read the last valid row (their results are not stored).
  // Offsets are 32-bit element offsets from the slab base pointers As / Bs,
  // which advance one slab per K step (the host checks they fit).
  constexpr int RSTEP = NT / 8;
  const int c0 = tid & 7, r0 = tid >> 3;
  uint32_t aoff[CONV ? 1 : ACH], boff[BCH];
  int32_t cvoff[CONV ? ACH : 1];
  uint32_t cvmask[CONV ? ACH : 1];
  if constexpr (CONV) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int m = min(m0 + r0 + RSTEP * i, M - 1);
      const int ow = m % cv.oW, t2 = m / cv.oW, oh = t2 % cv.oH, b = t2 / cv.oH;
      const int ih0 = oh * cv.s - cv.p, iw0 = ow * cv.s - cv.p;
      cvoff[i] = ((b * cv.iH + ih0) * cv.iW + iw0) * int(cv.ldx) * 2 + c0 * 16;
      uint32_t msk = 0;
      for (int kh = 0; kh < cv.kH; ++kh)
        for (int kw = 0; kw < cv.kW; ++kw)
          if (unsigned(ih0 + kh) < unsigned(cv.iH) && unsigned(iw0 + kw) < unsigned(cv.iW)) msk |= 1u << (kh * cv.kW + kw);
      cvmask[i] = msk;
    }
  } else {
#pragma unroll
    for (int i = 0; i < ACH; ++i) aoff[i] = uint32_t(min(m0 + r0 + RSTEP * i, M - 1)) * uint32_t(lda) + c0 * 8;
  }
#pragma unroll
  for (int i = 0; i < BCH; ++i) boff[i] = uint32_t(min(n0 + r0 + RSTEP * i, N - 1)) * uint32_t(ldb) + c0 * 8;
  // CONV slab state (wave-uniform): tap (kh, kw), first channel, and the
  // tap's byte offset from a row's tap (0, 0)
  const __amdgpu_buffer_rsrc_t xres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(A), 0, CONV ? cv.B * cv.iH * cv.iW * int(cv.ldx) * 2 : 0,
                                        0x00020000);
  int ckh = 0, ckw = 0, cic = 0, ctap = 0, csoff = 0;
  auto conv_next = [&]() {
    cic += 64;
    if (cic == cv.iC) {
      cic = 0;
      if (++ckw == cv.kW) {
        ckw = 0;
        ++ckh;
      }
      ctap = ckh * cv.kW + ckw;
    }
    csoff = ((ckh * cv.iW + ckw) * int(cv.ldx) + cic) * 2;
  };
  auto conv_chunk = [&](int i) -> u32x4 {
    const uint32_t voff = ((cvmask[i] >> ctap) & 1u) ? uint32_t(cvoff[i] + csoff) : 0x80000000u;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, voff, 0, 0));
  };
  const int sw = r0 * 8 + (c0 ^ (r0 & 7));  // row r0 + RSTEP * i sits at sw + RSTEP * 8 * i
  const uint16_t *As = A, *Bs = Bt;
  u32x4 ra[ACH], rb[BCH];
#define MH_PGLOAD()                                                                                \
  {                                                                                                \
    if constexpr (CONV) {                                                                          \
      _Pragma("unroll") for (int i = 0; i < ACH; ++i) ra[i] = conv_chunk(i);                       \
    } else {                                                                                       \
      _Pragma("unroll") for (int i = 0; i < ACH; ++i) ra[i] = ldg16(As + aoff[i]);                 \
    }                                                                                              \
    _Pragma("unroll") for (int i = 0; i < BCH; ++i) rb[i] = ldg16(Bs + boff[i]);                   \
  }
#define MH_PSTORE(L)                                                                               \
  {                                                                                                \
    _Pragma("unroll") for (int i = 0; i < ACH; ++i)(L)[sw + RSTEP * 8 * i] = ra[i];                \
    _Pragma("unroll") for (int i = 0; i < BCH; ++i)(L)[BM * 8 + sw + RSTEP * 8 * i] = rb[i];       \
  }
  f32x4 acc[FM][FN];
  u32x4 af0[FM], bf0[FN], af1[FM], bf1[FN];
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

  typedef PipeEpi<DT, BM, BN, WGM, WGN, EK> Epi;
  Epi epi(ep, g, M, N, m0, n0);
  epi.prefetch(ep);

  // slab 0 covers columns [0, K0), K0 = K % 64 (or 64): chunks at or past K0
  // are zero; every later slab is whole
  const int KT = (K + BK - 1) / BK, K0 = K - (KT - 1) * BK;
  u32x4 *L0 = lds[0], *L1 = lds[1];
  typename Epi::LnIn lnin;
  if constexpr (PipeKindT<EK>::LN) epi.ln_issue(ep, lnin, tid);
  if constexpr (CONV) {  // K % 64 == 0: slab 0 is whole
    MH_PGLOAD();
  } else {
    const bool cin = c0 * 8 < K0;
#pragma unroll
    for (int i = 0; i < ACH; ++i) ra[i] = cin ? ldg16(As + aoff[i]) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < BCH; ++i) rb[i] = cin ? ldg16(Bs + boff[i]) : u32x4{0, 0, 0, 0};
  }
  MH_PSTORE(L0);
  if constexpr (PipeKindT<EK>::LN) epi.ln_finish(ep, lnin, lnrow, lncs, lnbw, tid);
  if (KT == 1) {
    __syncthreads();
    g.template frags<0>(L0, af0, bf0);
    g.template frags<1>(L0, af1, bf1);
    MH_PMMA0(af0, bf0);
    MH_PMMA(af1, bf1);
  } else {
    if constexpr (CONV) conv_next();
    else As += K0;
    Bs += K0;
    MH_PGLOAD();
    __syncthreads();
    g.template frags<0>(L0, af0, bf0);
    // K step k: slab k in L0 with its first-half fragments in af0 / bf0, slab
    // k + 1 in the staging registers.  The loads of a step past the last slab
    // re-read the last slab (always whole, so in bounds); their data is stored
    // to the idle buffer and never read.  Step 0 is peeled: its first MFMAs
    // start the accumulators.
#define MH_PSTEP(KNEXT, MMAA)                                                                      \
  {                                                                                                \
    MH_PSTORE(L1);                                                                                 \
    if ((KNEXT) < KT) {                                                                            \
      if constexpr (CONV) conv_next();                                                             \
      else As += BK;                                                                               \
      Bs += BK;                                                                                    \
    }                                                                                              \
    MH_PGLOAD();                                                                                   \
    g.template frags<1>(L0, af1, bf1);                                                             \
    MMAA(af0, bf0);                                                                                \
    MH_SCHED_A();                                                                                  \
    __syncthreads();                                                                               \
    g.template frags<0>(L1, af0, bf0);                                                             \
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
#undef MH_SCHED_A
#undef MH_SCHED_B

  epi.store(ep, acc, ep.mode == EPI_ROWMAJOR ? z * sc : 0, &lds[0][0], wave, lane,
            PipeKindT<EK>::LN ? lnrow : nullptr, PipeKindT<EK>::LN ? lncs : nullptr,
            PipeKindT<EK>::LN ? lnbw : nullptr);
}

// ---- direct-to-LDS kernel ----

// vmcnt(N) only (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] |
// vmcnt[5:4] in [15:14]); inline assembly so that the wait-count pass keeps it
// exactly where it is.
template <int N> __device__ __forceinline__ void dma_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One wave instruction: 64 lanes x 16 bytes from base + voff (per lane) into
// LDS bytes [m0, m0 + 1024) (lane l at m0 + 16 l).
__device__ __forceinline__ void dma16(const uint16_t *base, uint32_t voff, uint32_t ldsaddr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(ldsaddr)
               : "memory", "m0");
}

// One wave instruction: 64 lanes x 16 bytes through a buffer resource into
// LDS bytes [m0, m0 + 1024): a lane whose offset lies past the resource's end
// writes zeros (the convolution's padding taps).
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t res, uint32_t voff, uint32_t ldsaddr) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(res), "s"(ldsaddr)
               : "memory", "m0");
}

// One wave instruction: 64 lanes x 4 bytes from base + voff into LDS bytes
// [m0, m0 + 256).
__device__ __forceinline__ void dma4(const void *base, uint32_t voff, uint32_t ldsaddr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(ldsaddr)
               : "memory", "m0");
}

// CONV: implicit-GEMM convolution (M = output pixels, N = oC, K = kH kW iC,
// iC % 64 == 0: slab kt is tap kt / (iC / 64) and 64 consecutive channels)
// on an NHWC activation A with OHWI weights Bt.  Each lane keeps, per A row
// it loads, the byte offset of the row's tap (0, 0) chunk and a bit mask of
// its taps inside the image; a slab's A blocks go straight to LDS through a
// buffer resource over the activation, padding taps reading an offset past
// its end (zeros), so the convolution runs the S-stage pipeline of the
// products.
template <int DT, int BM, int BN, int WGM, int WGN, int S, int EK, bool CONV = false>
__global__ void __launch_bounds__(WGM * WGN * 64)
gemm_dma_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ Bt, int M, int N, int K, long lda,
                long ldb, long sa, long sb, long sc, EpiArgs ep, ConvArgs cv = ConvArgs{}) {
  typedef PipeGeom<BM, BN, WGM, WGN> G;
  constexpr int NW = G::NW, FM = G::FM, FN = G::FN, BK = 64;
  // 8-row DMA blocks per wave per slab.  EVEN: every wave takes the same
  // number of A blocks and of Bt blocks.  Otherwise block b of the NB blocks
  // (A rows, then Bt rows) goes to wave b % NW, and a wave with one block
  // fewer repeats the slab's last block (the same bytes to the same LDS
  // address), so every wave issues NDMA instructions and waits for the same
  // counts.
  constexpr bool EVEN = BM % (8 * NW) == 0 && BN % (8 * NW) == 0;
  constexpr int NB = (BM + BN) / 8, NBA = BM / 8;
  constexpr int ABLK = EVEN ? BM / 8 / NW : 1, BBLK = EVEN ? BN / 8 / NW : 1;
  constexpr int NDMA = EVEN ? ABLK + BBLK : (NB + NW - 1) / NW;
  static_assert(BM % 8 == 0 && BN % 8 == 0, "DMA blocks");
  static_assert(S >= 2 && NDMA * (S - 1) < 64, "stages");
  static_assert(!CONV || EVEN, "convolution tiles split their DMA blocks evenly");
  constexpr uint32_t STAGE = (BM + BN) * 128;  // bytes per stage
  __shared__ u32x4 lds[S][(BM + BN) * 8];
  __shared__ float2 lnrow[BM];  // folded LayerNorm: row (mean, rstd)
  __shared__ __attribute__((aligned(16))) float lncs[BN], lnbw[BN];  // and column terms

  int m0, n0;
  pipe_tile<BM, BN>(M, N, ep.xcd_gn, m0, n0);
  const int z = blockIdx.z;
  A += z * sa;
  Bt += z * sb;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const G g(wave, lane);
  // lane l of a DMA instruction fetches block row l / 8, global chunk
  // (l % 8) ^ (l / 8): the chunk that the swizzle stores at LDS slot l.
  // Byte offsets from the slab base (rows past M / N read the last valid row).
  const int lr = lane >> 3, lc = (lane & 7) ^ lr;
  uint32_t aoff[ABLK], boff[BBLK];
  uint32_t uoff[EVEN ? 1 : NDMA];
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>((lds_void_t *)&lds[0][0]));
  int32_t cvoff[CONV ? ABLK : 1];
  uint32_t cvmask[CONV ? ABLK : 1];
  if constexpr (CONV) {
#pragma unroll
    for (int i = 0; i < ABLK; ++i) {
      const int m = min(m0 + (wave * ABLK + i) * 8 + lr, M - 1);
      const int ow = m % cv.oW, t2 = m / cv.oW, oh = t2 % cv.oH, b = t2 / cv.oH;
      const int ih0 = oh * cv.s - cv.p, iw0 = ow * cv.s - cv.p;
      cvoff[i] = ((b * cv.iH + ih0) * cv.iW + iw0) * int(cv.ldx) * 2 + lc * 16;
      uint32_t msk = 0;
      for (int kh = 0; kh < cv.kH; ++kh)
        for (int kw = 0; kw < cv.kW; ++kw)
          if (unsigned(ih0 + kh) < unsigned(cv.iH) && unsigned(iw0 + kw) < unsigned(cv.iW)) msk |= 1u << (kh * cv.kW + kw);
      cvmask[i] = msk;
    }
  }
  const __amdgpu_buffer_rsrc_t xres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(A), 0, CONV ? cv.B * cv.iH * cv.iW * int(cv.ldx) * 2 : 0,
                                        0x00020000);
  const int KT = K / BK;
  // Convolution: the slab the next DMAs fetch (wave-uniform): its index,
  // Bt slab pointer, tap (kh, kw), first channel and byte offset from a
  // row's tap (0, 0) chunk.  The DMAs fetch slabs in order (the prologue's,
  // then one per step, the last one again past the end), so the state steps
  // one slab after each slab's DMAs instead of being recomputed from the
  // slab index every step (two divisions: by the channel blocks per tap and
  // by the kernel width).  A plain GEMM computes its slab pointers from the
  // step index, which takes fewer scalar instructions than carrying them.
  int ckt = 0, ckh = 0, ckw = 0, cic = 0, ctap = 0, csoff = 0;
  const uint16_t *bsl = Bt;
  auto slab_adv = [&]() {
    if constexpr (CONV) {
      if (ckt + 1 >= KT) return;
      ++ckt;
      bsl += BK;
      cic += 64;
      if (cic == cv.iC) {
        cic = 0;
        if (++ckw == cv.kW) {
          ckw = 0;
          ++ckh;
        }
        ctap = ckh * cv.kW + ckw;
      }
      csoff = ((ckh * cv.iW + ckw) * int(cv.ldx) + cic) * 2;
    }
  };
  if constexpr (EVEN) {
#pragma unroll
    for (int i = 0; i < ABLK; ++i)
      aoff[i] = (uint32_t(min(m0 + (wave * ABLK + i) * 8 + lr, M - 1)) * uint32_t(lda) + lc * 8) * 2;
#pragma unroll
    for (int i = 0; i < BBLK; ++i)
      boff[i] = (uint32_t(min(n0 + (wave * BBLK + i) * 8 + lr, N - 1)) * uint32_t(ldb) + lc * 8) * 2;
  } else {
#pragma unroll
    for (int t = 0; t < NDMA; ++t) {
      const int b = min(wave + t * NW, NB - 1);
      uoff[t] = b < NBA ? (uint32_t(min(m0 + b * 8 + lr, M - 1)) * uint32_t(lda) + lc * 8) * 2
                        : (uint32_t(min(n0 + (b - NBA) * 8 + lr, N - 1)) * uint32_t(ldb) + lc * 8) * 2;
    }
  }
  const uint32_t wa = lds0 + wave * ABLK * 1024, wb = lds0 + BM * 128 + wave * BBLK * 1024;
  // DMA instruction t of slab kt into stage st (EVEN: A blocks first; else
  // block min(wave + t NW, NB - 1), whose LDS rows start at 1024 b bytes)
#define MH_DMA(T, KT_, ST)                                                                         \
  {                                                                                                \
    if constexpr (!EVEN) {                                                                         \
      const int b_ = min(wave + (T) * NW, NB - 1);                                                 \
      dma16((b_ < NBA ? A : Bt) + (KT_) * BK, uoff[(T) % NDMA], lds0 + (ST) * STAGE + b_ * 1024);  \
    } else if ((T) < ABLK) {                                                                       \
      if constexpr (CONV) {                                                                        \
        const uint32_t v_ = ((cvmask[(T) % ABLK] >> ctap) & 1u) ? uint32_t(cvoff[(T) % ABLK] + csoff) \
                                                                : 0x80000000u;                     \
        dma16_buf(xres, v_, wa + (ST) * STAGE + ((T) % ABLK) * 1024);                              \
      } else {                                                                                     \
        dma16(A + (KT_) * BK, aoff[(T) % ABLK], wa + (ST) * STAGE + ((T) % ABLK) * 1024);          \
      }                                                                                            \
    } else                                                                                         \
      dma16(CONV ? bsl : Bt + (KT_) * BK, boff[((T) - ABLK) % BBLK],                               \
            wb + (ST) * STAGE + (((T) - ABLK) % BBLK) * 1024);                                     \
  }

  f32x4 acc[FM][FN];
  u32x4 af0[FM], bf0[FN], af1[FM], bf1[FN];
  typedef PipeEpi<DT, BM, BN, WGM, WGN, EK> Epi;
  Epi epi(ep, g, M, N, m0, n0);
  // the next GEMM's weights: this workgroup's share of their 128-byte lines,
  // one 4-byte load each, issued first, into the first 256 bytes of the last
  // stage.  Every wave waits for its own loads (the oldest) before the first
  // barrier, and the last stage is first written (slab S - 1) and first read
  // only after that barrier, so no wave's prefetch can land on data that
  // another wave has written or will read (the LayerNorm row buffer, written
  // by every wave before the barrier, could be overwritten that way).
  if (ep.pf) {
    const uint32_t lines = uint32_t((ep.pf_bytes + 127) >> 7), nwg = gridDim.x * gridDim.z;
    const uint32_t per = min((lines + nwg - 1) / nwg, 4u * G::NT), first = (blockIdx.z * gridDim.x + blockIdx.x) * per;
    const uint32_t lsc = lds0 + (S - 1) * STAGE;
    for (uint32_t i = tid; i < per; i += G::NT)
      if (first + i < lines) dma4(ep.pf, (first + i) << 7, lsc);
  }
  // a fixed program's bias / residual prefetch goes after the first slabs'
  // loads, and the wait for slab 0 leaves it in flight (issued first, the
  // residual's scattered 8-byte loads held slab 0's wait back: 1.3 us of
  // the prologue on the 128x96 tile); the general program's load count is
  // known only at run time, so it prefetches first
  constexpr bool LATE_PRE = PipeKindT<EK>::FIXED;
  static_assert(NDMA * (S - 2) + Epi::NPRE < 64, "vmcnt range");
  if constexpr (!LATE_PRE) epi.prefetch(ep);

  typename Epi::LnIn lnin;
  if constexpr (PipeKindT<EK>::LN) epi.ln_issue(ep, lnin, tid);
  // prologue: slabs 0 .. S-2 in flight (re-loading the last slab past the
  // end), wait for slab 0
#pragma unroll
  for (int s = 0; s < S - 1; ++s) {
    const int kt = min(s, KT - 1);
#pragma unroll
    for (int t = 0; t < NDMA; ++t) MH_DMA(t, kt, s);
    slab_adv();
  }
  if constexpr (LATE_PRE) {
    epi.prefetch(ep);
    dma_wait<NDMA * (S - 2) + Epi::NPRE>();
  } else {
    dma_wait<NDMA * (S - 2)>();
  }
  if constexpr (PipeKindT<EK>::LN) epi.ln_finish(ep, lnin, lnrow, lncs, lnbw, tid);
  __syncthreads();
  g.template frags<0>(lds[0], af0, bf0);

  // Step k on stage s = k % S (a wave-uniform index: one step per loop trip
  // keeps every accumulator in one register assignment).  Phase A: each MFMA
  // of the first K half is followed by one DMA of slab k + S - 1 (into stage
  // (k + S - 1) % S), then by one fragment read of the second half; wait for
  // slab k + 1; barrier.  Phase B: each MFMA of the second half is followed by
  // one fragment read of slab k + 1's first half.  The order is written out
  // and pinned with sched_barrier (the scheduler cannot place inline assembly
  // in sched_group_barrier slots).
  constexpr int NMM = FM * FN, NRD = FM + FN;
  // Two stages: slab k + 1 is fetched during step k and read in step k's
  // second half.  Its wait and barrier come LATE MFMAs before the end of that
  // half (RPM fragment reads per MFMA after them) rather than at its start,
  // so the fetch has most of the step to land instead of half of it.  RPM =
  // 2 (3 and 5 measured the same).
  constexpr int RPM = 2;
  constexpr int LATE = S == 2 ? (NRD + RPM - 1) / RPM : 0;
  static_assert(LATE <= NMM, "late wait");
  constexpr int STAGE4 = (BM + BN) * 8;  // u32x4 per stage
  const int c1 = 4 + g.lg, c0f = g.lg;
#define MH_FRAG(L, C, X, AF, BF)                                                                   \
  {                                                                                                \
    if ((X) < FM) {                                                                                \
      const int r = g.wm * G::WTM + ((X) % FM) * 16 + g.li;                                        \
      AF[(X) % FM] = (L)[r * 8 + ((C) ^ (r & 7))];                                                 \
    } else {                                                                                       \
      const int r = g.wn * G::WTN + (((X) - FM) % FN) * 16 + g.li;                                 \
      BF[((X) - FM) % FN] = (L)[BM * 8 + r * 8 + ((C) ^ (r & 7))];                                 \
    }                                                                                              \
  }
  // stage of the current step: k % S, carried from step to step when S is
  // not a power of two (a remainder by 3 costs a multiply-high sequence of
  // scalar instructions every step)
  constexpr bool CARRY = (S & (S - 1)) != 0;
  int stg = 0;
#define MH_DSTEP(KK, FIRST)                                                                        \
  {                                                                                                \
    const int s_ = CARRY ? stg : (KK) % S, sn_ = s_ + 1 == S ? 0 : s_ + 1, sf_ = s_ == 0 ? S - 1 : s_ - 1; \
    const int kf_ = min((KK) + S - 1, KT - 1);                                                     \
    const u32x4 *Ls_ = &lds[0][0] + s_ * STAGE4, *Ln_ = &lds[0][0] + sn_ * STAGE4;                 \
    _Pragma("unroll") for (int t = 0; t < NMM; ++t) {                                              \
      if (FIRST) PipeMfma<DT>::mma0(acc[t / FN][t % FN], bf0[t % FN], af0[t / FN]);                \
      else PipeMfma<DT>::mma(acc[t / FN][t % FN], bf0[t % FN], af0[t / FN]);                       \
      if (t < NDMA) MH_DMA(t, kf_, sf_)                                                            \
      else if (t < NDMA + NRD) MH_FRAG(Ls_, c1, t - NDMA, af1, bf1)                                \
      __builtin_amdgcn_sched_barrier(0);                                                           \
    }                                                                                              \
    _Pragma("unroll") for (int t = NMM; t < NDMA + NRD; ++t) {                                     \
      if (t < NDMA) MH_DMA(t, kf_, sf_)                                                            \
      else MH_FRAG(Ls_, c1, t - NDMA, af1, bf1)                                                    \
    }                                                                                              \
    slab_adv();                                                                                    \
    if constexpr (LATE == 0) {                                                                     \
      dma_wait<NDMA * (S - 2)>();                                                                  \
      __syncthreads();                                                                             \
    }                                                                                              \
    _Pragma("unroll") for (int t = 0; t < NMM; ++t) {                                              \
      if (LATE > 0 && t == NMM - LATE) {                                                           \
        dma_wait<0>();                                                                             \
        __syncthreads();                                                                           \
      }                                                                                            \
      PipeMfma<DT>::mma(acc[t / FN][t % FN], bf1[t % FN], af1[t / FN]);                            \
      if (LATE == 0) {                                                                             \
        if (t < NRD) MH_FRAG(Ln_, c0f, t, af0, bf0)                                                \
      } else if (t >= NMM - LATE) {                                                                \
        _Pragma("unroll") for (int q_ = 0; q_ < RPM; ++q_)                                          \
          if (RPM * (t - (NMM - LATE)) + q_ < NRD) MH_FRAG(Ln_, c0f, RPM * (t - (NMM - LATE)) + q_, af0, bf0) \
      }                                                                                            \
      __builtin_amdgcn_sched_barrier(0);                                                           \
    }                                                                                              \
    if constexpr (LATE == 0) {                                                                     \
      _Pragma("unroll") for (int t = NMM; t < NRD; ++t) MH_FRAG(Ln_, c0f, t, af0, bf0)             \
    }                                                                                              \
    stg = sn_;                                                                                     \
  }
  MH_DSTEP(0, true);
  for (int k = 1; k < KT; ++k) MH_DSTEP(k, false);
#undef MH_DSTEP
#undef MH_DMA
#undef MH_FRAG
  // every load has landed and every wave is done with the stages before the
  // epilogue reuses the LDS or the workgroup ends
  dma_wait<0>();
  __syncthreads();
  epi.store(ep, acc, ep.mode == EPI_ROWMAJOR ? z * sc : 0, &lds[0][0], wave, lane,
            PipeKindT<EK>::LN ? lnrow : nullptr, PipeKindT<EK>::LN ? lncs : nullptr,
            PipeKindT<EK>::LN ? lnbw : nullptr);
}

#undef MH_PMMA
#undef MH_PMMA0

template <int DT, int BM, int BN, int WGM, int WGN, int EK = PK_GENERAL>
void launch(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa, long sb,
            long sc, const EpiArgs &ep, hipStream_t st) {
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_pipe_kernel<DT, BM, BN, WGM, WGN, EK>), dim3(tiles, 1, batch), dim3(WGM * WGN * 64), 0, st,
                     (const uint16_t *)A, (const uint16_t *)Bt, M, N, K, lda, ldb, sa, sb, sc, ep, ConvArgs{});
}

// implicit-GEMM convolution on the register-staged kernel (x NHWC, w OHWI)
template <int DT, int BM, int BN, int WGM, int WGN>
void launch_conv(const void *x, const void *w, const ConvArgs &cv, int oC, const EpiArgs &ep, hipStream_t st) {
  const int M = cv.B * cv.oH * cv.oW, K = cv.kH * cv.kW * cv.iC;
  const int tiles = ((M + BM - 1) / BM) * ((oC + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_pipe_kernel<DT, BM, BN, WGM, WGN, PK_GENERAL, true>), dim3(tiles), dim3(WGM * WGN * 64), 0,
                     st, (const uint16_t *)x, (const uint16_t *)w, M, oC, K, 0L, long(K), 0L, 0L, 0L, ep, cv);
}

template <int DT, int BM, int BN, int WGM, int WGN, int S, int EK = PK_GENERAL>
void launch_dma(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa, long sb,
                long sc, const EpiArgs &ep, hipStream_t st) {
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_dma_kernel<DT, BM, BN, WGM, WGN, S, EK>), dim3(tiles, 1, batch), dim3(WGM * WGN * 64), 0,
                     st, (const uint16_t *)A, (const uint16_t *)Bt, M, N, K, lda, ldb, sa, sb, sc, ep, ConvArgs{});
}

// implicit-GEMM convolution on the direct-to-LDS kernel (x NHWC, w OHWI)
template <int DT, int BM, int BN, int WGM, int WGN, int S>
void launch_dma_conv(const void *x, const void *w, const ConvArgs &cv, int oC, const EpiArgs &ep, hipStream_t st) {
  const int M = cv.B * cv.oH * cv.oW, K = cv.kH * cv.kW * cv.iC;
  const int tiles = ((M + BM - 1) / BM) * ((oC + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_dma_kernel<DT, BM, BN, WGM, WGN, S, PK_GENERAL, true>), dim3(tiles), dim3(WGM * WGN * 64),
                     0, st, (const uint16_t *)x, (const uint16_t *)w, M, oC, K, 0L, long(K), 0L, 0L, 0L, ep, cv);
}

}  // namespace

// Fixed epilogue programs (kind != PK_GENERAL; fp16: those without a folded
// LayerNorm) on the tiles the automatic choice uses: 0 128x128, 1 128x64, 2 64x64, 3 128x96
// (register-staged, gemm_pipe_fixed_staged.hip) and 8 128x96 4 stages,
// 9 128x128 2 stages (direct-to-LDS, gemm_pipe_fixed_dma.hip).  They return
// hipErrorNotSupported for any other tile.
hipError_t gemm_pipe_fixed_staged(int dt, int kind, int tile, const void *A, const void *Bt, int M, int N, int K, long lda,
                                  long ldb, int batch, long sa, long sb, long sc, const EpiArgs &ep, hipStream_t st);
// Eight-wave direct-to-LDS tiles, every program (gemm_pipe_wide.hip): 16
// 256x192 two stages, 17 128x96 four stages.
hipError_t gemm_pipe_wide(int dt, int kind, int tile, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb,
                          int batch, long sa, long sb, long sc, const EpiArgs &ep, hipStream_t st);
hipError_t gemm_pipe_fixed_dma(int dt, int kind, int tile, const void *A, const void *Bt, int M, int N, int K, long lda,
                               long ldb, int batch, long sa, long sb, long sc, const EpiArgs &ep, hipStream_t st);

}  // namespace mh
