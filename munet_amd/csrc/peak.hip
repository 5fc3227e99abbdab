// Measured peaks of this GPU.
//
// Matrix cores: every wave of a full grid issues
// independent v_mfma_f32_16x16x32_bf16 / _f16 instructions (the instruction
// of the GEMM and attention kernels) on register operands, with no memory
// traffic in the loop.  The roofline reports it beside the datasheet peak:
// it is what the clock sustains under an all-MFMA load.
#include "mh_common.hpp"
#include "mh_kernels.hpp"

namespace mh {

constexpr int kPeakAcc = 8;       // independent accumulators per wave
constexpr int kPeakBlocks = 2048; // 8 waves per CU on 256 CUs, 4 per block

// sink for the (never taken) store that keeps the accumulators live; a
// symbol the host could read, so the store is not dead
__device__ float mfma_peak_sink[kPeakBlocks];

namespace {

template <int DT>
__global__ void __launch_bounds__(256) mfma_peak_kernel(int iters, float seed) {
  typedef __attribute__((ext_vector_type(8))) short s8;
  s8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = short(int(seed * float(threadIdx.x + i)) & 0x3fff);
    b[i] = short(int(seed * float(i + 1)) & 0x3fff);
  }
  f32x4 acc[kPeakAcc];
#pragma unroll
  for (int j = 0; j < kPeakAcc; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kPeakAcc; ++j) {
      if constexpr (DT == BF16)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                        acc[j], 0, 0, 0);
      else
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                       acc[j], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kPeakAcc; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  if (s == 1234567.f) mfma_peak_sink[blockIdx.x] = s;
}

}  // namespace

hipError_t mfma_peak(int dt, int iters, double *flops_per_s, hipStream_t st) {
  if (iters <= 0 || !flops_per_s || (dt != BF16 && dt != F16)) return hipErrorInvalidValue;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t err = hipEventCreate(&e0);
  if (err == hipSuccess) err = hipEventCreate(&e1);
  auto launch = [&]() {
    if (dt == BF16)
      hipLaunchKernelGGL(mfma_peak_kernel<BF16>, dim3(kPeakBlocks), dim3(256), 0, st, iters, 1.0f);
    else
      hipLaunchKernelGGL(mfma_peak_kernel<F16>, dim3(kPeakBlocks), dim3(256), 0, st, iters, 1.0f);
    return hipGetLastError();
  };
  if (err == hipSuccess) err = launch();  // warm-up (clock ramp)
  if (err == hipSuccess) err = hipEventRecord(e0, st);
  if (err == hipSuccess) err = launch();
  if (err == hipSuccess) err = hipEventRecord(e1, st);
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  float ms = 0.f;
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (err != hipSuccess) return err;
  const double flops = double(kPeakBlocks) * 4 * iters * kPeakAcc * (16.0 * 16 * 32 * 2);
  *flops_per_s = ms > 0.f ? flops / (double(ms) * 1e-3) : 0.0;
  return hipSuccess;
}

// Measured HBM read rate: a full grid streams a caller's buffer (much larger
// than the last-level cache) with 16-byte loads, four in flight per thread,
// folding them into one value per thread so no load is dead.  Read-only: the
// roofline of a kernel that mostly reads is this rate, not a copy's.
constexpr int kReadBlocks = 8192;
__device__ int hbm_read_sink[kReadBlocks];

namespace {

typedef int i32x4v __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) hbm_read_kernel(const i32x4v *__restrict__ p, size_t n16) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  i32x4v acc = {0, 0, 0, 0};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const i32x4v a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= p[i];
  const int s = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (s == 0x5a5a5a5a) hbm_read_sink[blockIdx.x] = s;
}

}  // namespace

hipError_t hbm_read_rate(const void *buf, size_t bytes, int reps, double *bytes_per_s, hipStream_t st) {
  if (!buf || bytes < 16 || reps <= 0 || !bytes_per_s || (uintptr_t)buf % 16) return hipErrorInvalidValue;
  const size_t n16 = bytes / 16;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t err = hipEventCreate(&e0);
  if (err == hipSuccess) err = hipEventCreate(&e1);
  auto launch = [&]() {
    hipLaunchKernelGGL(hbm_read_kernel, dim3(kReadBlocks), dim3(256), 0, st, static_cast<const i32x4v *>(buf), n16);
    return hipGetLastError();
  };
  if (err == hipSuccess) err = launch();  // warm-up
  if (err == hipSuccess) err = hipEventRecord(e0, st);
  for (int r = 0; r < reps && err == hipSuccess; ++r) err = launch();
  if (err == hipSuccess) err = hipEventRecord(e1, st);
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  float ms = 0.f;
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (err != hipSuccess) return err;
  *bytes_per_s = ms > 0.f ? double(n16) * 16.0 * reps / (double(ms) * 1e-3) : 0.0;
  return hipSuccess;
}

}  // namespace mh
