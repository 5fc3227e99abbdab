// C ABI of libmunet_hip.so (declared in include/munet_hip.h).
//
// Thin layer: validate arguments, translate MuNet's capability-call
// arguments into launcher arguments, enqueue, and turn HIP failures into a
// non-zero status with a thread-local message (the C++ side above maps that
// to std::runtime_error, as MuNet's backends throw, reference
// src/backend/cuda_backend.cu:15-31 for the error convention).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/munet_hip.h"
#include "host_codec.hpp"
#include "mh_kernels.hpp"
#include "mh_runtime.hpp"

namespace mh {

void hip_check(hipError_t e, const char *what);

namespace {
thread_local std::string g_last_error;

struct DeviceState {
  int *err_flag = nullptr;  // device int, embedding index errors
  void *workspace = nullptr;
  size_t workspace_bytes = 0;
};
std::mutex g_mu;
std::unordered_map<int, DeviceState> g_devices;

// Fixed scratch for mh_matmul_noalloc: the operand transposes that mh_matmul
// stages in its growable workspace go here instead, so that entry point
// never allocates.  Each GPU the library runs on holds its own copy, at its
// own address, until the process ends.  In host code `scratch` names only
// the host-side shadow of the symbol; device addresses come from
// hipGetSymbolAddress, once per device, and are kept in g_scratch.
constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
void *g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The device address of `scratch` on `device` (the current device),
// resolved on first use and kept.
void *scratch_ptr(int device) {
  if (device < 0 || device >= kMaxDevices) throw Error("device ordinal out of range for the scratch table");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[device]) {
    void *ptr = nullptr;
    hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!ptr) throw Error("hipGetSymbolAddress(scratch) returned no address");
    g_scratch[device] = ptr;
  }
  return g_scratch[device];
}

void check_dt(int dt, bool allow_int = false) {
  if (dt < 0 || dt > 3 || (!allow_int && dt == 3)) throw Error("unsupported dtype code " + std::to_string(dt));
}
}  // namespace

void set_last_error(const std::string &msg) { g_last_error = msg; }

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

int current_device() {
  int d = 0;
  hip_check(hipGetDevice(&d), "hipGetDevice");
  return d;
}

static DeviceState &state() {
  const int d = current_device();
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState &s = g_devices[d];
  if (!s.err_flag) {
    hip_check(hipMalloc(&s.err_flag, sizeof(int)), "hipMalloc(error flag)");
    hip_check(hipMemset(s.err_flag, 0, sizeof(int)), "hipMemset(error flag)");
  }
  return s;
}

int *device_error_flag() { return state().err_flag; }

void *workspace(size_t bytes) {
  DeviceState &s = state();
  std::lock_guard<std::mutex> lk(g_mu);
  if (bytes > s.workspace_bytes) {
    if (s.workspace) {
      hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
      hip_check(hipFree(s.workspace), "hipFree(workspace)");
      s.workspace = nullptr;
    }
    const size_t rounded = (bytes + (1u << 20) - 1) & ~size_t((1u << 20) - 1);
    hip_check(hipMalloc(&s.workspace, rounded), "hipMalloc(workspace)");
    s.workspace_bytes = rounded;
  }
  return s.workspace;
}

static double g_last_kernel_us = 0.0;
void set_last_kernel_time_us(double us) { g_last_kernel_us = us; }

}  // namespace mh

using namespace mh;

#define MH_TRY(...)                                    \
  try {                                                \
    __VA_ARGS__;                                       \
    return 0;                                          \
  } catch (const std::exception &e) {                  \
    mh::set_last_error(e.what());                      \
    return 1;                                          \
  }

#define S_(p) static_cast<hipStream_t>(p)

namespace {

void bin_call(int dt, int op, const void *a, const void *b, void *out, int ndim, const int *shape, const int64_t *sa,
              const int64_t *sb, void *stream) {
  check_dt(dt);
  if (ndim < 0 || ndim > kMaxDims) throw Error("broadcast rank must be <= 6");
  BcastArgs g;
  g.ndim = ndim;
  g.total = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) throw Error("negative dimension");
    g.shape[d] = shape[d];
    g.sa[d] = long(sa[d]);
    g.sb[d] = long(sb[d]);
    g.total *= size_t(shape[d]);
  }
  hip_check(binary(dt, op, a, b, out, g, S_(stream)), "binary");
}

void un_call(int dt, int op, const void *in, void *out, size_t n, void *stream, float c = 0.f) {
  check_dt(dt);
  hip_check(unary(dt, op, in, out, n, c, S_(stream)), "unary");
}

// Bytes of transposed operands a matmul stages: A when transA, B when not
// transB (the NT GEMM reads A [M,K] and B as [N,K]), each slot 256-aligned.
size_t matmul_staging_bytes(int dt, int batch, int M, int K, int N, bool transA, bool transB, long sb) {
  const size_t es = dt_size(dt);
  const size_t nb_b = sb == 0 ? 1 : size_t(batch);
  size_t need = 0;
  if (transA) need += (size_t(batch) * M * K * es + 255) & ~size_t(255);
  if (!transB) need += (nb_b * K * N * es + 255) & ~size_t(255);
  return need;
}

void matmul_check(int dt, int batch, int M, int K, int N) {
  check_dt(dt);
  if (M < 0 || K < 0 || N < 0 || batch < 0) throw Error("matmul: negative size");
}

// A [M,K] (or [K,M] when transA) and B [K,N] (or [N,K] when transB) per
// batch slice -> the NT GEMM's operands, transposing into `ws` (at least
// matmul_staging_bytes, 256-byte aligned).
void matmul_staged(int dt, const void *a, const void *b, void *out, int batch, int M, int K, int N, bool transA,
                   bool transB, long sa, long sb, long sc, char *ws, void *stream) {
  const size_t es = dt_size(dt);
  const int nb_b = sb == 0 ? 1 : batch;
  const void *A = a, *Bt = b;
  long lsa = sa, lsb = sb;
  if (transA) {
    // per-slice [K,M] -> [M,K]; slices may be strided, so one launch each
    // unless they are packed back to back
    char *dst = ws;
    if (sa == long(M) * K || batch == 1) {
      hip_check(transpose2d(dt, a, dst, batch, K, M, S_(stream)), "transpose A");
    } else {
      for (int z = 0; z < batch; ++z)
        hip_check(transpose2d(dt, static_cast<const char *>(a) + size_t(z) * sa * es, dst + size_t(z) * M * K * es,
                              1, K, M, S_(stream)),
                  "transpose A");
    }
    A = dst;
    lsa = long(M) * K;
    ws += (size_t(batch) * M * K * es + 255) & ~size_t(255);
  }
  if (!transB) {
    char *dst = ws;
    if (sb == 0 || sb == long(K) * N || nb_b == 1) {
      hip_check(transpose2d(dt, b, dst, nb_b, K, N, S_(stream)), "transpose B");
    } else {
      for (int z = 0; z < nb_b; ++z)
        hip_check(transpose2d(dt, static_cast<const char *>(b) + size_t(z) * sb * es, dst + size_t(z) * K * N * es,
                              1, K, N, S_(stream)),
                  "transpose B");
    }
    Bt = dst;
    lsb = sb == 0 ? 0 : long(K) * N;
  }
  EpiArgs ep;
  ep.out = out;
  ep.ldc = N;
  hip_check(gemm_nt(dt, A, Bt, M, N, K, K, K, batch, lsa, lsb, sc, ep, -1, S_(stream)), "gemm");
}

void matmul_call(int dt, const void *a, const void *b, void *out, int batch, int M, int K, int N, bool transA,
                 bool transB, long sa, long sb, long sc, void *stream) {
  matmul_check(dt, batch, M, K, N);
  if (M == 0 || N == 0 || batch == 0) return;
  const size_t need = matmul_staging_bytes(dt, batch, M, K, N, transA, transB, sb);
  char *ws = need ? static_cast<char *>(workspace(need)) : nullptr;
  matmul_staged(dt, a, b, out, batch, M, K, N, transA, transB, sa, sb, sc, ws, stream);
}

}  // namespace

extern "C" {

const char *mh_last_error(void) { return mh::g_last_error.c_str(); }
const char *mh_version(void) { return "munet-hip 0.1 (gfx950)"; }

int mh_query_support(int feature, int dtype, int *available, int *fallback_policy, int *accumulation_dtype) {
  MH_TRY({
    check_dt(dtype, true);
    if (!available || !fallback_policy || !accumulation_dtype) throw Error("query_support: null output");
    const bool fp = dtype != MH_I32;
    bool ok = false;
    switch (feature) {
    // the float products, elementwise, activation, normalisation and spatial
    // kernels: fp32, fp16 and bf16 storages
    case MH_FEATURE_ELEMENTWISE_BINARY:
    case MH_FEATURE_MATMUL:
    case MH_FEATURE_UNARY_ACTIVATION:
    case MH_FEATURE_SOFTMAX:
    case MH_FEATURE_CONVOLUTION:
    case MH_FEATURE_POOLING:
    case MH_FEATURE_LAYER_NORM:
    case MH_FEATURE_ATTENTION:
    case MH_FEATURE_EMBEDDING:
    case MH_FEATURE_MASKED_FILL:
      ok = fp;
      break;
    // data movement: any storage, int32 included (broadcast_row runs as a
    // strided gather with a zero row stride)
    case MH_FEATURE_BROADCAST_ROW:
    case MH_FEATURE_CONCAT:
    case MH_FEATURE_TO_CONTIGUOUS:
      ok = true;
      break;
    // training-only capabilities and the reductions are not part of the
    // inference path: unavailable, never silently sent to the CPU
    default:
      ok = false;
      break;
    }
    *available = ok ? 1 : 0;
    *fallback_policy = MH_POLICY_EXPLICIT_UNSUPPORTED;
    *accumulation_dtype = MH_F32;
  })
}

int mh_device_count(int *count) {
  MH_TRY({
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
  })
}

int mh_init(int device) {
  MH_TRY({
    hip_check(hipSetDevice(device), "hipSetDevice");
    (void)state();
    (void)scratch_ptr(device);
  })
}

int mh_check_device_errors(void) {
  MH_TRY({
    int *flag = device_error_flag();
    int h = 0;
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    hip_check(hipMemcpy(&h, flag, sizeof(int), hipMemcpyDeviceToHost), "hipMemcpy(error flag)");
    if (h) {
      hip_check(hipMemset(flag, 0, sizeof(int)), "hipMemset(error flag)");
      if (h & 1) throw Error("Embedding index out of range");
      throw Error("device error flag set");
    }
  })
}

// ---- allocation / transfer -------------------------------------------------
int mh_allocate(void **ptr, size_t bytes) {
  MH_TRY({
    *ptr = nullptr;
    if (bytes) hip_check(hipMalloc(ptr, bytes), "hipMalloc");
  })
}
int mh_deallocate(void *ptr) { MH_TRY(if (ptr) hip_check(hipFree(ptr), "hipFree")) }
int mh_memset(void *ptr, int value, size_t bytes, void *stream) {
  MH_TRY(if (bytes) hip_check(hipMemsetAsync(ptr, value, bytes, S_(stream)), "hipMemsetAsync"))
}
int mh_copy(const void *src, void *dst, size_t bytes, int src_dev, int dst_dev, void *stream) {
  MH_TRY({
    if (bytes > 0 && (!src || !dst)) throw Error("hip copy: null pointer with non-zero byte count");
    if (!bytes) return 0;
    hipMemcpyKind kind;
    if (src_dev == MH_DEVICE_CPU && dst_dev == MH_DEVICE_CPU) kind = hipMemcpyHostToHost;
    else if (src_dev == MH_DEVICE_CPU) kind = hipMemcpyHostToDevice;
    else if (dst_dev == MH_DEVICE_CPU) kind = hipMemcpyDeviceToHost;
    else kind = hipMemcpyDeviceToDevice;
    hip_check(hipMemcpyAsync(dst, src, bytes, kind, S_(stream)), "hipMemcpyAsync");
    if (kind == hipMemcpyDeviceToHost || kind == hipMemcpyHostToDevice)
      hip_check(hipStreamSynchronize(S_(stream)), "hipStreamSynchronize");
  })
}
int mh_synchronize(void *stream) {
  MH_TRY({
    if (stream) hip_check(hipStreamSynchronize(S_(stream)), "hipStreamSynchronize");
    else hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  })
}
double mh_get_last_kernel_time_us(void) { return mh::g_last_kernel_us; }

int mh_to_contiguous(int dt, const void *src, void *dst, int ndim, const int *shape, const int64_t *strides,
                     int64_t offset, void *stream) {
  MH_TRY({
    check_dt(dt, true);
    if (ndim < 0 || ndim > kMaxDims) throw Error("to_contiguous: rank must be <= 6");
    StridedArgs g;
    g.ndim = ndim;
    g.offset = long(offset);
    g.total = 1;
    for (int d = 0; d < ndim; ++d) {
      g.shape[d] = shape[d];
      g.strides[d] = long(strides[d]);
      g.total *= size_t(shape[d]);
    }
    hip_check(to_contiguous(dt, src, dst, g, S_(stream)), "to_contiguous");
  })
}

// ---- elementwise -----------------------------------------------------------
int mh_add(int dt, const void *a, const void *b, void *out, int ndim, const int *shape, const int64_t *sa,
           const int64_t *sb, void *stream) {
  MH_TRY(bin_call(dt, BIN_ADD, a, b, out, ndim, shape, sa, sb, stream))
}
int mh_sub(int dt, const void *a, const void *b, void *out, int ndim, const int *shape, const int64_t *sa,
           const int64_t *sb, void *stream) {
  MH_TRY(bin_call(dt, BIN_SUB, a, b, out, ndim, shape, sa, sb, stream))
}
int mh_mul(int dt, const void *a, const void *b, void *out, int ndim, const int *shape, const int64_t *sa,
           const int64_t *sb, void *stream) {
  MH_TRY(bin_call(dt, BIN_MUL, a, b, out, ndim, shape, sa, sb, stream))
}
int mh_div(int dt, const void *a, const void *b, void *out, int ndim, const int *shape, const int64_t *sa,
           const int64_t *sb, void *stream) {
  MH_TRY(bin_call(dt, BIN_DIV, a, b, out, ndim, shape, sa, sb, stream))
}
int mh_relu(int dt, const void *in, void *out, size_t n, void *stream) { MH_TRY(un_call(dt, UN_RELU, in, out, n, stream)) }
int mh_sigmoid(int dt, const void *in, void *out, size_t n, void *stream) { MH_TRY(un_call(dt, UN_SIGMOID, in, out, n, stream)) }
int mh_exp(int dt, const void *in, void *out, size_t n, void *stream) { MH_TRY(un_call(dt, UN_EXP, in, out, n, stream)) }
int mh_log(int dt, const void *in, void *out, size_t n, void *stream) { MH_TRY(un_call(dt, UN_LOG, in, out, n, stream)) }
int mh_sqrt(int dt, const void *in, void *out, size_t n, void *stream) { MH_TRY(un_call(dt, UN_SQRT, in, out, n, stream)) }
int mh_rsqrt(int dt, const void *in, void *out, size_t n, void *stream) { MH_TRY(un_call(dt, UN_RSQRT, in, out, n, stream)) }
int mh_sin(int dt, const void *in, void *out, size_t n, void *stream) { MH_TRY(un_call(dt, UN_SIN, in, out, n, stream)) }
int mh_cos(int dt, const void *in, void *out, size_t n, void *stream) { MH_TRY(un_call(dt, UN_COS, in, out, n, stream)) }
int mh_gelu(int dt, const void *in, void *out, size_t n, void *stream) {
  MH_TRY(un_call(dt, UN_GELU, in, out, n, stream, host_round(dt, 1.702f)))
}
int mh_softmax(int dt, const void *in, void *out, int batch, int classes, void *stream) {
  MH_TRY({
    check_dt(dt);
    hip_check(softmax_rows(dt, in, out, batch, classes, S_(stream)), "softmax");
  })
}
int mh_masked_fill(int dt, const void *x, const int32_t *mask, void *out, size_t n, double value, void *stream) {
  MH_TRY({
    check_dt(dt);
    // the fill value is written through the dtype codec (-1e9 -> -inf in fp16)
    hip_check(masked_fill(dt, x, mask, out, n, float(value), S_(stream)), "masked_fill");
  })
}
int mh_layer_norm(int dt, const void *x, const void *w, const void *b, void *out, int rows, int cols, float eps,
                  void *stream) {
  MH_TRY({
    check_dt(dt);
    hip_check(layernorm(dt, x, w, b, out, rows, cols, eps, S_(stream)), "layer_norm");
  })
}
int mh_embedding(int dt, const int32_t *ids, const void *w, void *out, int n, int V, int D, void *stream) {
  MH_TRY({
    check_dt(dt);
    hip_check(embedding(dt, ids, w, nullptr, out, n, V, D, 1, device_error_flag(), S_(stream)), "embedding");
  })
}
int mh_embedding_pos(int dt, const int32_t *ids, const void *tok_w, const void *pos_w, void *out, int n, int V, int D,
                     int T, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (T <= 0) throw Error("embedding_pos: T must be positive");
    hip_check(embedding(dt, ids, tok_w, pos_w, out, n, V, D, T, device_error_flag(), S_(stream)), "embedding");
  })
}
int mh_convert(int sdt, const void *in, int ddt, void *out, size_t n, void *stream) {
  MH_TRY({
    check_dt(sdt, true);
    check_dt(ddt, true);
    hip_check(convert(sdt, in, ddt, out, n, S_(stream)), "convert");
  })
}
int mh_check_f16_rounding(unsigned long long *mismatches, void *stream) {
  MH_TRY({
    if (!mismatches) throw Error("check_f16_rounding: mismatches must be set");
    hip_check(check_f16_rounding(mismatches, S_(stream)), "check_f16_rounding");
  })
}
int mh_argmax(int dt, const void *x, int32_t *out, int rows, int cols, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (cols <= 0) throw Error("argmax: empty rows");
    hip_check(argmax_rows(dt, x, out, rows, cols, S_(stream)), "argmax");
  })
}
int mh_measure_mfma_peak(int dt, int iters, double *flops_per_s, void *stream) {
  MH_TRY({
    if (dt != MH_BF16 && dt != MH_F16) throw Error("measure_mfma_peak: dtype must be bfloat16 or float16");
    if (iters <= 0 || !flops_per_s) throw Error("measure_mfma_peak: iters must be positive and flops_per_s set");
    hip_check(mfma_peak(dt, iters, flops_per_s, S_(stream)), "measure_mfma_peak");
  })
}
int mh_measure_hbm_read(const void *buf, size_t bytes, int reps, double *bytes_per_s, void *stream) {
  MH_TRY({
    if (!buf || bytes < (size_t(1) << 20) || reps <= 0 || !bytes_per_s || (uintptr_t)buf % 16)
      throw Error("measure_hbm_read: needs a 16-byte aligned buffer of at least 1 MiB, reps > 0 and bytes_per_s");
    hip_check(hbm_read_rate(buf, bytes, reps, bytes_per_s, S_(stream)), "measure_hbm_read");
  })
}

// ---- blas ------------------------------------------------------------------
int mh_matmul(int dt, const void *a, const void *b, void *out, int M, int K, int N, int transA, int transB,
              void *stream) {
  MH_TRY(matmul_call(dt, a, b, out, 1, M, K, N, transA != 0, transB != 0, 0, 0, 0, stream))
}
int mh_matmul_noalloc(int dt, const void *a, const void *b, void *out, int M, int K, int N, int transA, int transB,
                      void *stream) {
  MH_TRY({
    matmul_check(dt, 1, M, K, N);
    if (M == 0 || N == 0) return 0;
    const size_t need = matmul_staging_bytes(dt, 1, M, K, N, transA != 0, transB != 0, 0);
    if (need > kScratchBytes)
      throw Error("matmul_noalloc: the transposed operands need " + std::to_string(need) + " bytes of scratch, " +
                  "more than its fixed " + std::to_string(kScratchBytes) + " bytes");
    char *ws = nullptr;
    if (need) {
      int dev = 0;
      hip_check(hipGetDevice(&dev), "hipGetDevice");
      ws = static_cast<char *>(scratch_ptr(dev));
    }
    matmul_staged(dt, a, b, out, 1, M, K, N, transA != 0, transB != 0, 0, 0, 0, ws, stream);
  })
}
int mh_batched_matmul(int dt, const void *a, const void *b, void *out, int batch, int M, int K, int N, int transA,
                      int transB, int64_t sa, int64_t sb, int64_t sc, void *stream) {
  MH_TRY(matmul_call(dt, a, b, out, batch, M, K, N, transA != 0, transB != 0, long(sa), long(sb), long(sc), stream))
}
int mh_linear(int dt, const void *x, const void *w_t, const void *bias, void *out, int M, int K, int N, int act,
              const void *resid, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (act < 0 || act > 2) throw Error("linear: bad activation code");
    EpiArgs ep;
    ep.out = out;
    ep.ldc = N;
    ep.bias = bias;
    ep.act = act;
    ep.gelu_c = host_round(dt, 1.702f);
    ep.resid = resid;
    ep.ldr = N;
    hip_check(gemm_nt(dt, x, w_t, M, N, K, K, K, 1, 0, 0, 0, ep, -1, S_(stream)), "linear");
  })
}
int mh_pack_linear_weight(int dt, const void *w, void *w_t, int in_f, int out_f, void *stream) {
  MH_TRY({
    check_dt(dt);
    hip_check(transpose2d(dt, w, w_t, 1, in_f, out_f, S_(stream)), "pack_linear_weight");
  })
}
int mh_qkv_projection(int dt, const void *x, const void *wqkv_t, const void *bqkv, void *q, void *k, void *v, int B,
                      int T, int E, int H, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (H <= 0 || E % H != 0) throw Error("qkv_projection: embed_dim must be divisible by num_heads");
    const int hd = E / H;
    if (hd % 4 != 0) throw Error("qkv_projection: head_dim must be a multiple of 4");
    EpiArgs ep;
    ep.mode = EPI_HEADSPLIT;
    ep.outs[0] = q;
    ep.outs[1] = k;
    ep.outs[2] = v;
    ep.bias = bqkv;
    ep.T = T;
    ep.H = H;
    ep.hd = hd;
    ep.E = E;
    hip_check(gemm_nt(dt, x, wqkv_t, B * T, 3 * E, E, E, E, 1, 0, 0, 0, ep, -1, S_(stream)), "qkv_projection");
  })
}

// ---- attention ---------------------------------------------------------------
int mh_attention(int dt, const void *q, const void *k, const void *v, void *ctx, int B, int H, int T, int hd,
                 int causal, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (hd <= 0) throw Error("attention: head_dim must be positive");
    if (size_t(T) * 4 > 64 * 1024 && !(hd == 64 && dt != MH_F32))
      throw Error("attention: sequence too long for the generic kernel");
    const float scale = host_round(dt, 1.0f / std::sqrt(float(hd)));
    hip_check(attention(dt, q, k, v, ctx, B, H, T, hd, causal, scale, 0, S_(stream)), "attention");
  })
}

int mh_attention_textbook(int dt, const void *q, const void *k, const void *v, void *ctx, int B, int H, int T, int hd,
                          int causal, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (hd <= 0) throw Error("attention: head_dim must be positive");
    if (size_t(T) * 4 > 64 * 1024 && !(hd == 64 && dt != MH_F32))
      throw Error("attention: sequence too long for the generic kernel");
    const float scale = host_round(dt, 1.0f / std::sqrt(float(hd)));
    hip_check(attention(dt, q, k, v, ctx, B, H, T, hd, causal, scale, 0, S_(stream), 1), "attention_textbook");
  })
}

// ---- shape -------------------------------------------------------------------
int mh_concat(int dt, const void *const *inputs, int count, void *out, int dim, int ndim, const int *shapes,
              void *stream) {
  MH_TRY({
    check_dt(dt, true);
    if (count <= 0) throw Error("concat: no inputs");
    if (dim < 0 || dim >= ndim) throw Error("concat: dim out of range");
    for (int j = 1; j < count; ++j)
      for (int d = 0; d < ndim; ++d)
        if (d != dim && shapes[j * ndim + d] != shapes[d]) throw Error("concat: shape mismatch");
    size_t outer = 1, inner = 1, total = 0;
    for (int d = 0; d < dim; ++d) outer *= size_t(shapes[d]);
    for (int d = dim + 1; d < ndim; ++d) inner *= size_t(shapes[d]);
    for (int j = 0; j < count; ++j) total += size_t(shapes[j * ndim + dim]);
    size_t off = 0;
    for (int j = 0; j < count; ++j) {
      const size_t len = size_t(shapes[j * ndim + dim]) * inner;
      hip_check(concat_part(dt, inputs[j], out, outer, len, total * inner, off, S_(stream)), "concat");
      off += len;
    }
  })
}
int mh_transpose2d(int dt, const void *in, void *out, int batch, int rows, int cols, void *stream) {
  MH_TRY({
    check_dt(dt, true);
    hip_check(transpose2d(dt, in, out, batch, rows, cols, S_(stream)), "transpose2d");
  })
}

// ---- spatial -----------------------------------------------------------------
static void conv_geom(ConvArgs &cv, int B, int iC, int iH, int iW, int kH, int kW, int s, int p) {
  if (s <= 0 || p < 0 || kH <= 0 || kW <= 0) throw Error("conv2d: bad stride/padding/kernel");
  cv.B = B; cv.iC = iC; cv.iH = iH; cv.iW = iW; cv.kH = kH; cv.kW = kW; cv.s = s; cv.p = p;
  cv.oH = (iH + 2 * p - kH) / s + 1;
  cv.oW = (iW + 2 * p - kW) / s + 1;
  cv.ldx = iC;
  if (cv.oH <= 0 || cv.oW <= 0) throw Error("conv2d: empty output");
}

int mh_pack_conv_weight(int dt, const void *w, void *w_ohwi, int oC, int iC, int kH, int kW, void *stream) {
  MH_TRY({
    check_dt(dt);
    hip_check(transpose2d(dt, w, w_ohwi, oC, iC, kH * kW, S_(stream)), "pack_conv_weight");
  })
}

int mh_conv2d_nhwc(int dt, const void *x, const void *w_ohwi, const void *bias, void *out, int B, int iC, int iH,
                   int iW, int oC, int kH, int kW, int s, int p, int act, void *stream) {
  MH_TRY({
    check_dt(dt);
    ConvArgs cv;
    conv_geom(cv, B, iC, iH, iW, kH, kW, s, p);
    EpiArgs ep;
    ep.out = out;
    ep.ldc = oC;
    ep.bias = bias;
    ep.bias_first = 1;
    ep.act = act;
    hip_check(conv_nhwc(dt, x, w_ohwi, cv, oC, ep, -1, S_(stream)), "conv2d_nhwc");
  })
}

int mh_conv2d(int dt, const void *in, const void *w, const void *bias, void *out, int B, int iC, int iH, int iW,
              int oC, int kH, int kW, int s, int p, void *stream) {
  MH_TRY({
    check_dt(dt);
    ConvArgs cv;
    conv_geom(cv, B, iC, iH, iW, kH, kW, s, p);
    const size_t es = dt_size(dt);
    const size_t xb = (size_t(B) * iC * iH * iW * es + 255) & ~size_t(255);
    const size_t wb = (size_t(oC) * iC * kH * kW * es + 255) & ~size_t(255);
    const size_t ob = size_t(B) * oC * cv.oH * cv.oW * es;
    char *ws = static_cast<char *>(workspace(xb + wb + ob + 256));
    hip_check(nchw_to_nhwc(dt, in, ws, B, iC, iH * iW, S_(stream)), "nchw_to_nhwc");
    hip_check(transpose2d(dt, w, ws + xb, oC, iC, kH * kW, S_(stream)), "pack weight");
    EpiArgs ep;
    ep.out = ws + xb + wb;
    ep.ldc = oC;
    ep.bias = bias;
    ep.bias_first = 1;
    hip_check(conv_nhwc(dt, ws, ws + xb, cv, oC, ep, -1, S_(stream)), "conv2d");
    hip_check(nhwc_to_nchw(dt, ws + xb + wb, out, B, oC, cv.oH * cv.oW, S_(stream)), "nhwc_to_nchw");
  })
}

int mh_pack_convt_weight(int dt, const void *w, void *w_packed, int iC, int oC, int k, void *stream) {
  MH_TRY({
    check_dt(dt);
    // out [kh][kw][oc][ic] gathered from in [ic][oc][kh][kw]
    StridedArgs g;
    g.ndim = 4;
    g.shape[0] = k; g.shape[1] = k; g.shape[2] = oC; g.shape[3] = iC;
    g.strides[0] = k; g.strides[1] = 1; g.strides[2] = long(k) * k; g.strides[3] = long(oC) * k * k;
    g.total = size_t(k) * k * oC * iC;
    hip_check(to_contiguous(dt, w, w_packed, g, S_(stream)), "pack_convt_weight");
  })
}

int mh_conv_transpose2d_nhwc(int dt, const void *x, const void *w_packed, const void *bias, void *out, int B, int iC,
                             int iH, int iW, int oC, int k, int64_t ldc, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (oC % 4 != 0) throw Error("conv_transpose2d: out channels must be a multiple of 4");
    if (ldc < oC) throw Error("conv_transpose2d: ldc < out channels");
    EpiArgs ep;
    ep.mode = EPI_CONVT;
    ep.out = out;
    ep.ldc = long(ldc);
    ep.bias = bias;
    ep.bias_first = 1;
    ep.convt_oc = oC;
    ep.convt_k = k;
    ep.convt_ih = iH;
    ep.convt_iw = iW;
    hip_check(gemm_nt(dt, x, w_packed, B * iH * iW, k * k * oC, iC, iC, iC, 1, 0, 0, 0, ep, -1, S_(stream)),
              "conv_transpose2d");
  })
}

int mh_max_pool2d(int dt, const void *in, void *out, int B, int C, int iH, int iW, int k, int s, int p, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (k <= 0 || s <= 0 || p < 0) throw Error("max_pool2d: bad window");
    hip_check(max_pool2d(dt, 0, in, out, B, C, iH, iW, k, s, p, S_(stream)), "max_pool2d");
  })
}
int mh_max_pool2d_nhwc(int dt, const void *in, void *out, int B, int C, int iH, int iW, int k, int s, int p,
                       void *stream) {
  MH_TRY({
    check_dt(dt);
    if (k <= 0 || s <= 0 || p < 0) throw Error("max_pool2d: bad window");
    hip_check(max_pool2d(dt, 1, in, out, B, C, iH, iW, k, s, p, S_(stream)), "max_pool2d_nhwc");
  })
}
int mh_upsample2d(int dt, const void *in, void *out, int B, int C, int iH, int iW, int scale, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (scale <= 0) throw Error("upsample2d: bad scale");
    hip_check(upsample2d(dt, 0, in, out, B, C, iH, iW, scale, S_(stream)), "upsample2d");
  })
}
int mh_upsample2d_nhwc(int dt, const void *in, void *out, int B, int C, int iH, int iW, int scale, void *stream) {
  MH_TRY({
    check_dt(dt);
    if (scale <= 0) throw Error("upsample2d: bad scale");
    hip_check(upsample2d(dt, 1, in, out, B, C, iH, iW, scale, S_(stream)), "upsample2d_nhwc");
  })
}
int mh_nchw_to_nhwc(int dt, const void *in, void *out, int B, int C, int HW, void *stream) {
  MH_TRY({
    check_dt(dt, true);
    hip_check(nchw_to_nhwc(dt, in, out, B, C, HW, S_(stream)), "nchw_to_nhwc");
  })
}
int mh_nhwc_to_nchw(int dt, const void *in, void *out, int B, int C, int HW, void *stream) {
  MH_TRY({
    check_dt(dt, true);
    hip_check(nhwc_to_nchw(dt, in, out, B, C, HW, S_(stream)), "nhwc_to_nchw");
  })
}

}  // extern "C"
