// Small fp32 products (ops::matmul / nn::Linear, reference
// src/core/ops/matmul.cpp:331-392, src/nn/linear.hpp:28-34, with the fused
// epilogue chain): the MLP and CNN classifiers, M <= 256 rows and few output
// tiles, where a 64x64 tile grid leaves most CUs idle and each K step of a
// tile waits a full memory latency.
//
// One workgroup per 16x16 output tile; its W waves split K into contiguous
// ranges of 16-wide groups.  Lane l loads, per group g, the 16 bytes
// A[m0 + l % 16][16 g + 4 (l / 16) .. + 3] and the same of Bt's row
// n0 + l % 16, and one v_mfma_f32_16x16x4f32 per element j takes element j
// of every lane: over the four MFMAs each lane's four K values meet their
// partners, so a group's 16 K values are summed with one 16-byte load per
// operand and lane (K is contracted in a permuted order, which a sum allows).
// A wave's groups are loaded in chunks of CH (8, or 4 with 16 waves, whose
// lanes have at most 128 VGPRs), the next chunk in flight while the current
// one is multiplied; the waves' partial tiles are added through
// LDS in wave order (deterministic) and the epilogue runs from wave 0.  With
// Bt as the first MFMA operand each lane ends with four consecutive output
// columns of one row, the layout of epi_store4.
#include "gemm_common.hpp"
#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {
namespace {

template <int W, int CH>
__global__ void __launch_bounds__(64 * W) gemm_skinny_kernel(const float *__restrict__ A, const float *__restrict__ Bt,
                                                             int M, int N, int K, long lda, long ldb, int gpw,
                                                             EpiArgs ep) {
  __shared__ f32x4 red[W][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.x * 16, n0 = blockIdx.y * 16;
  const int G = (K + 15) / 16;
  const int g0 = wave * gpw, g1 = min(g0 + gpw, G);
  const float *ar = A + long(min(m0 + li, M - 1)) * lda;
  const float *br = Bt + long(min(n0 + li, N - 1)) * ldb;
  // two register buffers, each indexed only by compile-time values (a
  // runtime buffer index put both in scratch)
  uint4 a0[CH], b0[CH], a1[CH], b1[CH];
  auto fetch = [&](uint4 (&ab)[CH], uint4 (&bb)[CH], int gs) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int k = 16 * (gs + i) + 4 * q;
      const bool in = gs + i < g1 && k < K;
      ab[i] = in ? *reinterpret_cast<const uint4 *>(ar + k) : make_uint4(0, 0, 0, 0);
      bb[i] = in ? *reinterpret_cast<const uint4 *>(br + k) : make_uint4(0, 0, 0, 0);
    }
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const uint4 (&ab)[CH], const uint4 (&bb)[CH]) {
#pragma unroll
    for (int i = 0; i < CH; ++i) Mfma<F32>::step(acc, bb[i], ab[i]);
  };
  if (g0 < g1) fetch(a0, b0, g0);
  for (int gs = g0; gs < g1; gs += 2 * CH) {
    if (gs + CH < g1) fetch(a1, b1, gs + CH);
    mma(a0, b0);
    if (gs + CH >= g1) break;
    if (gs + 2 * CH < g1) fetch(a0, b0, gs + 2 * CH);
    mma(a1, b1);
  }
  if constexpr (W > 1) {
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    acc = red[0][lane];
#pragma unroll
    for (int w = 1; w < W; ++w) acc += red[w][lane];
  }
  const int m = m0 + li, n = n0 + 4 * q;
  if (m < M && n < N) {
    float v[4] = {acc[0], acc[1], acc[2], acc[3]};
    epi_store4<F32>(ep, m, n, N, v, 0);
  }
}

}  // namespace

bool gemm_skinny_ok(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                    const EpiArgs &ep) {
  const long tiles = long((M + 15) / 16) * ((N + 15) / 16);
  // K <= 2048: longer products put too few workgroups on too many bytes
  // each (CNN 32 x 4096 -> 128: 16 workgroups, 18-21 us against 11.4 us for
  // the 64-slice split-K pair); they keep split-K
  return dt == F32 && batch == 1 && M > 0 && N > 0 && K >= 16 && K <= 2048 && M <= 256 && tiles <= 1024 && K % 4 == 0 &&
         lda % 4 == 0 && ldb % 4 == 0 && lda >= K && ldb >= K && (uintptr_t)A % 16 == 0 && (uintptr_t)Bt % 16 == 0 &&
         ep.mode == EPI_ROWMAJOR && !ep.stats_out && !ep.ln_stats;
}

hipError_t gemm_skinny(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, const EpiArgs &ep,
                       hipStream_t st) {
  const int G = (K + 15) / 16;
  // waves per tile: enough that each wave loads at most two chunks of 8
  // (at most 16 waves), then more while a wave still loads more than one
  // chunk and the grid holds fewer than 512 waves
  int W = 1;
  while (W < 16 && (G + W - 1) / W > 16) W *= 2;
  while (W < 16 && (G + W - 1) / W > 8 && long((M + 15) / 16) * ((N + 15) / 16) * W < 512) W *= 2;
  const int gpw = (G + W - 1) / W;
  const dim3 grid(unsigned((M + 15) / 16), unsigned((N + 15) / 16));
  const float *a = static_cast<const float *>(A), *b = static_cast<const float *>(Bt);
  switch (W) {
  case 1: hipLaunchKernelGGL((gemm_skinny_kernel<1, 8>), grid, dim3(64), 0, st, a, b, M, N, K, lda, ldb, gpw, ep); break;
  case 2: hipLaunchKernelGGL((gemm_skinny_kernel<2, 8>), grid, dim3(128), 0, st, a, b, M, N, K, lda, ldb, gpw, ep); break;
  case 4: hipLaunchKernelGGL((gemm_skinny_kernel<4, 8>), grid, dim3(256), 0, st, a, b, M, N, K, lda, ldb, gpw, ep); break;
  case 8: hipLaunchKernelGGL((gemm_skinny_kernel<8, 8>), grid, dim3(512), 0, st, a, b, M, N, K, lda, ldb, gpw, ep); break;
  default: hipLaunchKernelGGL((gemm_skinny_kernel<16, 4>), grid, dim3(1024), 0, st, a, b, M, N, K, lda, ldb, gpw, ep); break;
  }
  return hipGetLastError();
}

}  // namespace mh
