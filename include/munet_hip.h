/* C ABI of the MuNet MI355X (gfx950) HIP backend: libmunet_hip.so.
 *
 * Every entry point takes plain device pointers, sizes and an optional HIP
 * stream (`stream` = NULL means the HIP null stream), returns 0 on success and
 * a non-zero status otherwise; mh_last_error() gives the message of the last
 * failure on the calling thread.  No entry point allocates on the hot path
 * except where noted ("workspace"): those grow a per-device scratch buffer
 * on first use and must not be called under stream capture.
 *
 * Storage dtypes (MuNet DataType, reference src/types.hpp:16):
 *   0 = float32, 1 = float16, 2 = bfloat16, 3 = int32.
 * fp16 rounding is round-half-away (src/types.hpp:239-278), bf16 is RNE
 * without a NaN case (src/types.hpp:311-317), exactly as MuNet's codecs.
 *
 * Each declaration names the reference interface it replaces. */
#ifndef MUNET_HIP_H
#define MUNET_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MH_F32 0
#define MH_F16 1
#define MH_BF16 2
#define MH_I32 3

#define MH_DEVICE_CPU 0
#define MH_DEVICE_HIP 1

#define MH_ACT_NONE 0
#define MH_ACT_RELU 1
#define MH_ACT_GELU 2

/* ---- status / runtime --------------------------------------------------- */
/* Message of the last failed call on this thread ("" if none). */
const char *mh_last_error(void);
/* Library version string. */
const char *mh_version(void);
/* Number of visible HIP devices (BackendRegistry probe,
 * src/backend/backend_manager.cpp:21-42). */
int mh_device_count(int *count);
/* Select `device` for the calling thread and create its state. */
int mh_init(int device);
/* Backend::query_support (src/core/backend.hpp:411-425): whether this backend
 * runs `feature` on storages of `dtype`, the fallback policy when it does
 * not, and the accumulation dtype it prefers.  Feature codes 0-12 are the
 * reference's BackendFeature values in its order (src/core/backend.hpp:
 * 16-30); codes from 100 are the path's functions that have no reference
 * capability.  Policy codes follow BackendFallbackPolicy (:32-36): nothing
 * falls back to the CPU here, so the policy is always ExplicitUnsupported.
 * An unknown feature is unavailable (the reference's default); an unknown
 * dtype code is an error.  Needs no device. */
#define MH_FEATURE_ELEMENTWISE_BINARY 0
#define MH_FEATURE_BROADCAST_ROW 1
#define MH_FEATURE_MATMUL 2
#define MH_FEATURE_UNARY_ACTIVATION 3
#define MH_FEATURE_SOFTMAX 4
#define MH_FEATURE_CONCAT 5
#define MH_FEATURE_LOSS 6
#define MH_FEATURE_CONVOLUTION 7
#define MH_FEATURE_POOLING 8
#define MH_FEATURE_BATCH_NORM 9
#define MH_FEATURE_OPTIMIZER_STEP 10
#define MH_FEATURE_RANDOM_FILL 11
#define MH_FEATURE_REDUCTION 12
#define MH_FEATURE_TO_CONTIGUOUS 100
#define MH_FEATURE_LAYER_NORM 101
#define MH_FEATURE_ATTENTION 102
#define MH_FEATURE_EMBEDDING 103
#define MH_FEATURE_MASKED_FILL 104
#define MH_POLICY_EXPLICIT_UNSUPPORTED 0
#define MH_POLICY_CPU_FALLBACK 1
#define MH_POLICY_CONVERSION_FALLBACK 2
int mh_query_support(int feature, int dtype, int *available, int *fallback_policy, int *accumulation_dtype);
/* Poll and clear device-side error flags (embedding ids out of range);
 * synchronises the device.  Returns non-zero with a message if any was set. */
int mh_check_device_errors(void);

/* ---- BackendAllocationTransferCapability (src/core/backend.hpp:190-205) --- */
int mh_allocate(void **ptr, size_t bytes);                    /* :193 allocate */
int mh_deallocate(void *ptr);                                 /* :194 deallocate */
int mh_memset(void *ptr, int value, size_t bytes, void *stream); /* :195 memset */
/* :196-197 copy(src, dst, bytes, src_dev, dst_dev); devices MH_DEVICE_*.
 * Device-to-host copies complete before returning (MuNet copies are
 * synchronous, src/backend/cpu_backend.hpp:212-232). */
int mh_copy(const void *src, void *dst, size_t bytes, int src_dev, int dst_dev, void *stream);
int mh_synchronize(void *stream);                             /* :198 synchronize */
/* :200-201 get_last_kernel_time_us: GPU time of the last timed region. */
double mh_get_last_kernel_time_us(void);
/* :202-204 to_contiguous(src, dst, shape, strides, offset): strided gather. */
int mh_to_contiguous(int dt, const void *src, void *dst, int ndim, const int *shape, const int64_t *strides,
                     int64_t offset, void *stream);

/* ---- BackendElementwiseCapability (src/core/backend.hpp:207-238) --------- */
/* :210-217 add/sub/mul/div(a, b, out, BroadcastInfo): out_shape and the
 * per-operand element strides of compute_broadcast (src/types.hpp:436-478). */
int mh_add(int dt, const void *a, const void *b, void *out, int ndim, const int *out_shape,
           const int64_t *strides_a, const int64_t *strides_b, void *stream);
int mh_sub(int dt, const void *a, const void *b, void *out, int ndim, const int *out_shape,
           const int64_t *strides_a, const int64_t *strides_b, void *stream);
int mh_mul(int dt, const void *a, const void *b, void *out, int ndim, const int *out_shape,
           const int64_t *strides_a, const int64_t *strides_b, void *stream);
int mh_div(int dt, const void *a, const void *b, void *out, int ndim, const int *out_shape,
           const int64_t *strides_a, const int64_t *strides_b, void *stream);
int mh_relu(int dt, const void *in, void *out, size_t n, void *stream);    /* :220 */
int mh_sigmoid(int dt, const void *in, void *out, size_t n, void *stream); /* :222 */
int mh_exp(int dt, const void *in, void *out, size_t n, void *stream);     /* :226 */
int mh_log(int dt, const void *in, void *out, size_t n, void *stream);     /* :227 */
int mh_sqrt(int dt, const void *in, void *out, size_t n, void *stream);    /* :228 */
int mh_rsqrt(int dt, const void *in, void *out, size_t n, void *stream);   /* :229 */
int mh_sin(int dt, const void *in, void *out, size_t n, void *stream);     /* :230 */
int mh_cos(int dt, const void *in, void *out, size_t n, void *stream);     /* :231 */
/* :233-234 softmax(in, out, batch_size, num_classes): last-dim softmax. */
int mh_softmax(int dt, const void *in, void *out, int batch_size, int num_classes, void *stream);

/* ---- op-layer functions with no backend hook in the reference ------------ */
/* nn::GELU (src/nn/activations.hpp:31-38): x*sigmoid(x*1.702), three rounded ops. */
int mh_gelu(int dt, const void *in, void *out, size_t n, void *stream);
/* ops::masked_fill (src/core/ops/elementwise.cpp:8-53), int32 mask. */
int mh_masked_fill(int dt, const void *x, const int32_t *mask, void *out, size_t n, double value, void *stream);
/* ops::layer_norm (src/core/ops/normalization.cpp:125-224) over the last dim. */
int mh_layer_norm(int dt, const void *x, const void *weight, const void *bias, void *out, int rows, int cols,
                  float eps, void *stream);
/* nn::Embedding gather path (src/nn/linear.hpp:92-128): ids [n] int32,
 * weight [V, D].  Out-of-range ids write zeros and raise the device error
 * flag reported by mh_check_device_errors. */
int mh_embedding(int dt, const int32_t *ids, const void *weight, void *out, int n, int V, int D, void *stream);
/* Fused token + position embedding: out[r] = tok_w[ids[r]] + pos_w[r % T]
 * (two nn::Embedding gathers and ops::add, one rounding). */
int mh_embedding_pos(int dt, const int32_t *ids, const void *tok_w, const void *pos_w, void *out, int n, int V,
                     int D, int T, void *stream);
/* Tensor::to(DataType) (src/tensor.cpp:249-284) on device memory. */
int mh_convert(int src_dt, const void *in, int dst_dt, void *out, size_t n, void *stream);
/* No counterpart in the reference: a self-check of the kernels' fast fp16
 * rounding (zero and the normal half range by a bit trick, the rest by the
 * full codec that mh_convert uses) against that codec over all 2^32 float
 * bit patterns; *mismatches receives the count of patterns that differ in any
 * bit (0 when the fast path is exact).  Synchronises `stream`. */
int mh_check_f16_rounding(unsigned long long *mismatches, void *stream);
/* Row argmax, first index of the maximum (the demos' np.argmax). */
int mh_argmax(int dt, const void *x, int32_t *out, int rows, int cols, void *stream);
/* Measured matrix-core peak of this GPU in FLOP/s: a full grid of waves
 * issuing independent 16x16x32 bf16 (dt MH_BF16) or fp16 MFMAs on registers,
 * `iters` loop trips of 8 per wave, timed with HIP events on `stream` (the
 * call synchronises it).  No counterpart in the reference: the measured peak
 * that the roofline reports beside the datasheet one. */
int mh_measure_mfma_peak(int dt, int iters, double *flops_per_s, void *stream);
/* Measured HBM read rate in bytes/s: a full grid streams the caller's device
 * buffer `buf` (16-byte aligned, `bytes` >= 1 MiB; make it several times the
 * 256 MB last-level cache) `reps` times with 16-byte loads, timed with HIP
 * events on `stream` (the call synchronises it).  No counterpart in the
 * reference: the measured read peak the roofline reports beside the
 * datasheet HBM figure. */
int mh_measure_hbm_read(const void *buf, size_t bytes, int reps, double *bytes_per_s, void *stream);

/* ---- BackendBlasCapability (src/core/backend.hpp:250-260) ---------------- */
/* :253-254 matmul(a, b, out, M, K, N, transA, transB) on raw row-major storage.
 * Uses the workspace when transA or !transB. */
int mh_matmul(int dt, const void *a, const void *b, void *out, int M, int K, int N, int transA, int transB,
              void *stream);
/* No counterpart in the reference: mh_matmul for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as mh_matmul,
 * but the transposed operands it stages (A when transA, B when !transB) go to
 * a fixed 64 MiB per-device scratch array inside the library instead of the
 * growable workspace; a call needing more fails with a message and enqueues
 * nothing.  No hipMalloc/hipFree on any path.  The array's device address is
 * resolved by mh_init (or on the first call on a device).  Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 * two threads) race and must be serialised by the caller. */
int mh_matmul_noalloc(int dt, const void *a, const void *b, void *out, int M, int K, int N, int transA, int transB,
                      void *stream);
/* :255-259 batched_matmul(..., stride_a, stride_b, stride_out); stride_b = 0
 * broadcasts one right operand.  Workspace as mh_matmul. */
int mh_batched_matmul(int dt, const void *a, const void *b, void *out, int batch, int M, int K, int N, int transA,
                      int transB, int64_t stride_a, int64_t stride_b, int64_t stride_out, void *stream);
/* nn::Linear forward (src/nn/linear.hpp:28-34) with the weight pre-packed as
 * w_t [N, K] (mh_pack_linear_weight): out = act(x*W + bias) (+ resid), with
 * the reference's rounding after the matmul, the bias add, each GELU op and
 * the residual add.  bias / resid may be NULL; act is MH_ACT_*. */
int mh_linear(int dt, const void *x, const void *w_t, const void *bias, void *out, int M, int K, int N, int act,
              const void *resid, void *stream);
/* Repack a Linear weight [in, out] (MuNet layout, src/nn/linear.hpp:14) to
 * the K-contiguous [out, in] panel the MFMA GEMM reads. */
int mh_pack_linear_weight(int dt, const void *w, void *w_t, int in_features, int out_features, void *stream);
/* The q/k/v projections of nn::MultiHeadAttention with their permute to
 * [B, H, T, hd] (src/nn/attention.hpp:47-62) as one GEMM: wqkv_t [3E, E]
 * (rows q, k, v), bqkv [3E]; q/k/v outputs [B*H*T*hd]. */
int mh_qkv_projection(int dt, const void *x, const void *wqkv_t, const void *bqkv, void *q, void *k, void *v, int B,
                      int T, int E, int H, void *stream);

/* ---- fused attention (src/nn/attention.hpp:64-99) ------------------------- */
/* q, k, v in [B*H, T, hd] (permuted, contiguous); k is read as MuNet reads it:
 * its buffer viewed as a row-major [hd, B*H*T] matrix.  ctx is written merged
 * as [B, T, H*hd].  Scale = 1/sqrt(hd) rounded to dt. */
int mh_attention(int dt, const void *q, const void *k, const void *v, void *ctx, int B, int H, int T, int hd,
                 int causal, void *stream);
/* No counterpart in the reference (its attention has no per-position keys,
 * so it cannot be decoded incrementally): the same rounding steps with key j
 * of head (b, h) read as row (b*H + h)*T + j of k, like v.  The attention of
 * the KV-cache decode (mh_decoder_*) and of DecoderLM configs with
 * "attention": "textbook". */
int mh_attention_textbook(int dt, const void *q, const void *k, const void *v, void *ctx, int B, int H, int T,
                          int hd, int causal, void *stream);

/* ---- BackendShapeCapability (src/core/backend.hpp:263-271) --------------- */
/* :266-267 concat(inputs, out, dim, shapes): `count` contiguous inputs of rank
 * ndim, shapes row-major count x ndim. */
int mh_concat(int dt, const void *const *inputs, int count, void *out, int dim, int ndim, const int *shapes,
              void *stream);
/* out[b][c][r] = in[b][r][c] for batch slices of rows x cols. */
int mh_transpose2d(int dt, const void *in, void *out, int batch, int rows, int cols, void *stream);

/* ---- BackendSpatialCapability (src/core/backend.hpp:291-311) ------------- */
/* :294-296 conv2d(in, weight, bias, out, B, iC, iH, iW, oC, kH, kW, s, p):
 * NCHW / OIHW, bias may be NULL.  Workspace (layout change to NHWC). */
int mh_conv2d(int dt, const void *in, const void *weight, const void *bias, void *out, int B, int iC, int iH, int iW,
              int oC, int kH, int kW, int s, int p, void *stream);
/* Channels-last conv with OHWI weights (mh_pack_conv_weight); act fused. */
int mh_conv2d_nhwc(int dt, const void *x, const void *w_ohwi, const void *bias, void *out, int B, int iC, int iH,
                   int iW, int oC, int kH, int kW, int s, int p, int act, void *stream);
/* OIHW -> OHWI repack. */
int mh_pack_conv_weight(int dt, const void *w_oihw, void *w_ohwi, int oC, int iC, int kH, int kW, void *stream);
/* Transposed conv with kernel == stride (no overlap), NHWC in/out; weight
 * packed [k*k*oC, iC] by mh_pack_convt_weight; out row stride ldc >= oC lets
 * the result land inside a channel-concat buffer. */
int mh_conv_transpose2d_nhwc(int dt, const void *x, const void *w_packed, const void *bias, void *out, int B, int iC,
                             int iH, int iW, int oC, int k, int64_t ldc, void *stream);
/* [iC, oC, k, k] -> [k, k, oC, iC]. */
int mh_pack_convt_weight(int dt, const void *w, void *w_packed, int iC, int oC, int k, void *stream);
/* :302-303 max_pool2d(in, out, B, C, iH, iW, k, s, p), NCHW. */
int mh_max_pool2d(int dt, const void *in, void *out, int B, int C, int iH, int iW, int k, int s, int p, void *stream);
int mh_max_pool2d_nhwc(int dt, const void *in, void *out, int B, int C, int iH, int iW, int k, int s, int p,
                       void *stream);
/* :307-308 upsample2d(in, out, B, C, iH, iW, scale), nearest, NCHW. */
int mh_upsample2d(int dt, const void *in, void *out, int B, int C, int iH, int iW, int scale, void *stream);
int mh_upsample2d_nhwc(int dt, const void *in, void *out, int B, int C, int iH, int iW, int scale, void *stream);
/* Layout change between NCHW and NHWC. */
int mh_nchw_to_nhwc(int dt, const void *in, void *out, int B, int C, int HW, void *stream);
int mh_nhwc_to_nchw(int dt, const void *in, void *out, int B, int C, int HW, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MUNET_HIP_H */
