// Internal launcher declarations shared by the kernel translation units and
// the C-ABI layer.  Every launcher enqueues on the given stream and returns
// the launch status; shapes have been validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mh {

// Storage dtype codes (MuNet DataType order, reference src/types.hpp:16).
enum DType : int { F32 = 0, F16 = 1, BF16 = 2, I32 = 3 };

enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU = 2 };
enum EpiMode : int { EPI_ROWMAJOR = 0, EPI_HEADSPLIT = 1, EPI_CONVT = 2 };
enum BinOp : int { BIN_ADD = 0, BIN_SUB = 1, BIN_MUL = 2, BIN_DIV = 3 };
enum UnOp : int {
  UN_RELU = 0, UN_SIGMOID = 1, UN_GELU = 2, UN_EXP = 3, UN_LOG = 4,
  UN_SQRT = 5, UN_RSQRT = 6, UN_SIN = 7, UN_COS = 8
};

constexpr int kMaxDims = 6;

// Fused GEMM epilogue.
//   row-major : out[m*ldc + n]
//   head split: column n of a [M, nsplit*E] product goes to outs[n / E] in
//               [B, H, T, hd] order with m = b*T + t and n % E = h*hd + d
//   convT     : column n = (kh*k + kw)*oC + oc of input pixel m = (b, ih, iw)
//               goes to NHWC pixel (b, ih*k+kh, iw*k+kw), channel oc
// bias_first adds the bias to the fp32 accumulator before the single output
// rounding (convolution semantics); otherwise the Linear chain
// round(round(acc) + bias) is applied.
struct EpiArgs {
  void *out = nullptr;
  long ldc = 0;
  const void *bias = nullptr;   // [N] (or [oC] for convT) in the storage dtype
  int bias_first = 0;
  const void *resid = nullptr;  // [M, ldr] added after the activation
  long ldr = 0;
  int act = ACT_NONE;
  float gelu_c = 1.702f;        // GELU constant already rounded to the dtype
  int mode = EPI_ROWMAJOR;
  void *outs[3] = {nullptr, nullptr, nullptr};
  int T = 1, H = 1, hd = 1, E = 1;
  int convt_oc = 1, convt_k = 1, convt_ih = 1, convt_iw = 1;
  // LayerNorm folded across a GEMM boundary (bf16 pipelined kernels only):
  //   stats_out: the producer writes, for output row m and column group g of
  //     stats_cols columns (16, 32, 48 or 64), (mean, M2) of the group's
  //     rounded output values (M2 = sum of squared deviations from that
  //     mean) at stats_out[2 * (m * (N / stats_cols) + g)];
  //   ln_stats: the consumer's A rows are raw LayerNorm inputs x with
  //     ln_parts such partials of ln_cols columns per row
  //     (K = ln_cols * ln_parts), and its weights hold gamma (.) W; the
  //     product becomes LN(x) W as rstd_m * (acc - mean_m * ln_cs[n]) +
  //     ln_bw[n], with ln_cs the column sums of the folded weights and
  //     ln_bw = beta W, before the epilogue chain.
  float *stats_out = nullptr;
  int stats_cols = 16;
  const float *ln_stats = nullptr, *ln_cs = nullptr, *ln_bw = nullptr;
  int ln_parts = 0, ln_cols = 16;
  float ln_eps = 1e-5f;
  // pipelined GEMMs: tile columns per group of the per-XCD tile enumeration
  // (0: groups of 8 tile rows instead); set by the GEMM launcher
  int xcd_gn = 0;
  // the output is read by no kernel (the engine's final output, copied out
  // later): the bias epilogue stores it with non-temporal stores, so it does
  // not sit in the caches for the next forward's kernels to write back
  int stream_out = 0;
  // the next GEMM's weights (direct-to-LDS kernels): each workgroup touches
  // its share of these bytes, one 4-byte load per 128-byte line, before its
  // own loads, so they come from the memory-side cache instead of HBM when
  // that GEMM starts (0 bytes or more than 16 MiB: nothing)
  const void *pf = nullptr;
  long pf_bytes = 0;
};

// Implicit-GEMM convolution geometry (NHWC activation, ldx = pixel stride).
struct ConvArgs {
  int B = 0, iC = 0, iH = 0, iW = 0, kH = 1, kW = 1, s = 1, p = 0, oH = 0, oW = 0;
  long ldx = 0;
};

struct BcastArgs {
  int ndim = 0;
  int shape[kMaxDims] = {};
  long sa[kMaxDims] = {};
  long sb[kMaxDims] = {};
  size_t total = 0;
};

struct StridedArgs {
  int ndim = 0;
  int shape[kMaxDims] = {};
  long strides[kMaxDims] = {};
  long offset = 0;
  size_t total = 0;
};

// C = A[M,K] (row stride lda) * Bt[N,K]^T (row stride ldb), batch slices at
// element strides sa/sb/sc (sb = 0 broadcasts one weight).  tile_hint < 0
// picks the block tile automatically.
hipError_t gemm_nt(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                   long sa, long sb, long sc, const EpiArgs &ep, int tile_hint, hipStream_t st);
// Direct-to-LDS pipeline for aligned 16-bit operands (K % 64 == 0);
// tile: 0 256x256, 1 256x128, 2 128x256, 3 128x128, 4 128x64.
bool gemm_dma_ok(int dt, const void *A, const void *Bt, int K, long lda, long ldb, long sa, long sb);
hipError_t gemm_dma(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch, long sa,
                    long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st);
// Pipelined kernels for 16-bit aligned operands (K % 8 == 0, 16-byte aligned
// rows); tile: < 0 automatic; register-staged 0 128x128, 1 128x64, 2 64x64,
// 3 128x96; direct-to-LDS (K % 64 == 0, else 128x128 register-staged)
// 7 128x128 3 stages, 8 128x96 4 stages, 9 128x128 2 stages, 10 128x96
// 2 stages, 11 128x96 3 stages, 12 128x64 3 stages; eight waves 16 256x192
// 2 stages, 17 128x96 4 stages, 19 128x288 3 stages.
bool gemm_pipe_ok(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, long sa, long sb);
bool gemm_pipe_dma_ok(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb);
hipError_t gemm_pipe(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                     long sa, long sb, long sc, const EpiArgs &ep, int tile, hipStream_t st);
// Implicit-GEMM convolution on the register-staged pipelined kernel
// (gemm_pipe_conv.hip): 16-bit, NHWC x and OHWI w 16-byte aligned, iC % 64
// == 0, ldx % 8 == 0, at most 32 taps, every byte offset of x below 2^31.
bool gemm_pipe_conv_ok(int dt, const void *x, const void *w, const ConvArgs &cv);
hipError_t gemm_pipe_conv(int dt, const void *x, const void *w, const ConvArgs &cv, int oC, const EpiArgs &ep,
                          hipStream_t st);
// A 3x3 stride-1 pad-1 convolution of a 16-bit NCHW image with C <= 3
// channels into an NHWC activation (w32: the OIHW rows zero-padded to 32;
// ep: row-major output, bias_first), and a 1x1 convolution of an NHWC
// activation (iC 32 / 64 / 128 channels, rows of ldx) to oC <= 8 channels
// written NCHW (w: [oC][iC], bias [oC], act none or ReLU).
bool conv3x3_fewc_ok(int dt, int C, int k, int s, int p, int oC);
hipError_t conv3x3_fewc(int dt, const void *x, const void *w32, int B, int C, int H, int W, int oC, const EpiArgs &ep,
                        hipStream_t st);
bool conv1x1_nchw_ok(int dt, int iC, long ldx, int oC);
hipError_t conv1x1_nchw(int dt, const void *x, const void *w, const void *bias, void *out, long M, int HW, int iC,
                        long ldx, int oC, int act, hipStream_t st);
// fp32 C = A Bt^T for M <= 256 rows and at most 1024 16x16 output tiles (the
// small Linears): one workgroup per tile, K split over its waves, summed in
// wave order; the general epilogue chain.
bool gemm_skinny_ok(int dt, const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, int batch,
                    const EpiArgs &ep);
hipError_t gemm_skinny(const void *A, const void *Bt, int M, int N, int K, long lda, long ldb, const EpiArgs &ep,
                       hipStream_t st);
hipError_t conv_nhwc(int dt, const void *x, const void *w_ohwi, const ConvArgs &cv, int oC, const EpiArgs &ep,
                     int tile_hint, hipStream_t st);
// Split-K for small fp32 products (gemm.hip): the slice count for M x N x K
// (1: no split), and the product itself through an fp32 workspace of
// S * M * N floats (row-major epilogue only).
int splitk_count(int dt, int M, int N, int K);
hipError_t gemm_splitk(int dt, const void *A, const void *Bt, int M, int N, int K, int S, float *ws, const EpiArgs &ep,
                       hipStream_t st);

// Fused attention core (q, k, v in the head-split [B*H, T, hd] layout).
// textbook = 0: MuNet's scores, k's buffer read as a [hd, B*H*T] matrix;
// textbook = 1: key j of a head is row j of its k (the decode attention).
hipError_t attention(int dt, const void *q, const void *k, const void *v, void *ctx, int B, int H, int T, int hd,
                     int causal, float scale, int force_generic, hipStream_t st, int textbook = 0);

// KV-cache decode (decode.hip).  state: device ints {pos, step, pending}:
// the position of the tokens being fed, the index of the next generated
// token in `tokens`, and 1 while the head's greedy choices in best still have
// to be fed back.
// The step's first kernel: pending choices become ids / tokens[step] (best
// reset, position and step + 1), then the token + position rows of ids.
hipError_t dec_embed(int dt, int32_t *ids, unsigned long long *best, int32_t *tokens, int *state, const void *tok,
                     const void *pos_tab, void *out, int B, int V, int D, int cap, int *err, hipStream_t st);
// One weight-streaming Linear over M <= 16 rows (dec_linear kinds: 0
// LayerNorm + q/k/v, k and v into the caches at pos; 1 + residual; 2
// LayerNorm + GELU; 3 LayerNorm + greedy argmax folded into best; 4 the
// attention's per-block shares part_o / part_ml combined into the input,
// + residual).
struct DecLinear {
  const void *x = nullptr, *w = nullptr, *bias = nullptr, *ln_w = nullptr, *ln_b = nullptr, *resid = nullptr;
  const float *part_o = nullptr;
  const float2 *part_ml = nullptr;
  void *out = nullptr, *kc = nullptr, *vc = nullptr;
  unsigned long long *best = nullptr;
  const int *state = nullptr;
  int *pending = nullptr;  // kind 3: set to 1 once the choices are in best
  int M = 0, N = 0, K = 0, E = 0, H = 1, hd = 1, Lmax = 1, nsplit = 1;
  float eps = 1e-5f, gelu_c = 1.702f;
};
hipError_t dec_linear(int dt, int kind, const DecLinear &p, hipStream_t st);
// Keys per decode attention block.
constexpr int kDecKeyBlock = 256;
// One block per 256 keys of each head, blocks 0..blocks-1 (keys 0..256
// blocks - 1, which must hold the position; blocks <= ceil(Lmax / 256) <= 16):
// shares part_o [B*H][blocks][hd], part_ml [B*H][blocks]
hipError_t dec_attention(int dt, const void *q, const void *kc, const void *vc, const int *state, float *part_o,
                         float2 *part_ml, int B, int H, int hd, int Lmax, int blocks, float scale, hipStream_t st);
// When choices are pending: best [B] -> ids [B] and tokens[step] (best
// reset), position and step + 1 (after the last step of a call)
hipError_t dec_finish(unsigned long long *best, int32_t *ids, int32_t *tokens, int *state, int B, int cap,
                      hipStream_t st);
hipError_t kv_store(int dt, const void *k, const void *v, void *kc, void *vc, int BH, int T, int hd, int Lmax,
                    hipStream_t st);

hipError_t binary(int dt, int op, const void *a, const void *b, void *out, const BcastArgs &g, hipStream_t st);
hipError_t unary(int dt, int op, const void *in, void *out, size_t n, float c, hipStream_t st);
hipError_t masked_fill(int dt, const void *x, const int32_t *mask, void *out, size_t n, float value, hipStream_t st);
hipError_t convert(int sdt, const void *in, int ddt, void *out, size_t n, hipStream_t st);
// the fast fp16 rounding against the full codec over all 2^32 float bit
// patterns (synchronises st)
hipError_t check_f16_rounding(unsigned long long *mismatches, hipStream_t st);
// stats (optional): the LayerNorm statistics of each output row, one
// (mean, M2) partial over all D columns (the stats_out layout of EpiArgs with
// stats_cols = D).
hipError_t embedding(int dt, const int32_t *ids, const void *w, const void *pos, void *out, int n, int V, int D,
                     int T, int *err, hipStream_t st, float *stats = nullptr);
hipError_t argmax_rows(int dt, const void *x, int32_t *out, int rows, int cols, hipStream_t st);
// Measured matrix-core peak (peak.hip): FLOP/s of a full grid of independent
// 16x16x32 MFMAs (bf16 or fp16), `iters` loop trips per wave.
hipError_t mfma_peak(int dt, int iters, double *flops_per_s, hipStream_t st);
hipError_t hbm_read_rate(const void *buf, size_t bytes, int reps, double *bytes_per_s, hipStream_t st);

hipError_t layernorm(int dt, const void *x, const void *w, const void *b, void *y, int rows, int cols, float eps,
                     hipStream_t st);
hipError_t softmax_rows(int dt, const void *x, void *y, int rows, int cols, hipStream_t st);

hipError_t to_contiguous(int dt, const void *src, void *dst, const StridedArgs &g, hipStream_t st);
hipError_t transpose2d(int dt, const void *in, void *out, int batch, int rows, int cols, hipStream_t st);
hipError_t concat_part(int dt, const void *src, void *dst, size_t outer, size_t len, size_t out_len, size_t off,
                       hipStream_t st);
hipError_t max_pool2d(int dt, int nhwc, const void *in, void *out, int B, int C, int iH, int iW, int k, int s, int p,
                      hipStream_t st);
hipError_t upsample2d(int dt, int nhwc, const void *in, void *out, int B, int C, int iH, int iW, int scale,
                      hipStream_t st);
hipError_t nchw_to_nhwc(int dt, const void *in, void *out, int B, int C, int HW, hipStream_t st);
// NCHW [B, C, HW] -> NHWC [B, HW, Cp], channels C .. Cp-1 written as zero
hipError_t nchw_to_nhwc_pad(int dt, const void *in, void *out, int B, int C, int HW, int Cp, hipStream_t st);
hipError_t nhwc_to_nchw(int dt, const void *in, void *out, int B, int C, int HW, hipStream_t st);

inline size_t dt_size(int dt) { return (dt == 1 || dt == 2) ? 2 : 4; }

}  // namespace mh
