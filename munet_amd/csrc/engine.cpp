// Compiled inference executor for the HIP backend (C ABI in
// include/munet_hip_engine.h).
//
// The reference's inference::Engine (src/inference.hpp:292-801) runs the
// module tree eagerly op by op; its compile() is a shape contract plus warm-up
// forwards (src/inference.hpp:446-537) and every op output is a fresh
// allocation (src/backend/cpu_backend.hpp:188-209).  This executor keeps the
// same load / compile / run contract and, at compile time:
//   1. traces the module tree (reference nn:: semantics per module) into a
//      linear op list over SSA values;
//   2. fuses: GEMM + bias + ReLU/GELU (+ residual) epilogues, conv + bias +
//      ReLU, q/k/v projections into one head-splitting GEMM, token + position
//      embedding + add, UNet skip concats into zero-copy channel slices, and
//      (bf16) each transformer LayerNorm into the Linear after it (fold_ln);
//   3. plans every activation into one device arena by liveness intervals
//      (greedy best-offset placement, largest first); weights live in a
//      second arena packed into the kernels' K-contiguous layouts;
//   4. captures the whole forward into a hipGraph on one stream.
// run() is then one H2D copy, one graph launch and one D2H copy.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <memory>
#include <iomanip>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/munet_hip.h"
#include "../../include/munet_hip_engine.h"
#include "host_codec.hpp"
#include "json.hpp"
#include "mh_kernels.hpp"
#include "mh_runtime.hpp"

namespace mh {
namespace {

using Shape = std::vector<int>;

size_t numel(const Shape &s) {
  size_t n = 1;
  for (int d : s) n *= size_t(d);
  return n;
}

std::string shape_str(const Shape &s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? "," : "") + std::to_string(s[i]);
  return r + "]";
}

enum Layout { ROWMAJOR = 0, NHWC = 1 };

struct Val {
  Shape shape;   // logical shape (NCHW order for 4-D tensors even when stored NHWC)
  int dt = F32;
  int layout = ROWMAJOR;
  int alias_of = -1;   // value whose buffer this one lives in
  long alias_off = 0;  // element offset inside that buffer
  long row_stride = 0; // NHWC channel-slice views: elements between pixels
  int def = -1, last = -1;
  long offset = -1;    // byte offset in the arena (resolved through aliases)
  size_t bytes() const { return numel(shape) * dt_size(dt); }
};

// OP_CONV a[9]: the layouts it reads and writes
enum ConvLayout { CONV_NHWC = 0, CONV_NCHW_IN = 1, CONV_NCHW_OUT = 2 };

enum OpKind {
  OP_GEMM, OP_QKV, OP_ATTN, OP_LN, OP_EMBED, OP_EMBED_POS, OP_CONV, OP_CONVT, OP_POOL, OP_UPSAMPLE,
  OP_UNARY, OP_BINARY, OP_SOFTMAX, OP_TO_NHWC, OP_TO_NCHW
};

const char *op_name(int k) {
  static const char *n[] = {"gemm", "qkv_gemm", "attention", "layer_norm", "embedding", "embedding_pos", "conv2d",
                            "conv_transpose2d", "max_pool2d", "upsample2d", "unary", "binary", "softmax",
                            "nchw_to_nhwc", "nhwc_to_nchw"};
  return n[k];
}

struct Op {
  int kind;
  std::string name;
  std::vector<int> in, out;
  // integer attributes (meaning per kind)
  long a[12] = {0};
  float f = 0.f;
  const void *w = nullptr, *b = nullptr, *w2 = nullptr;
  int act = ACT_NONE;
  int resid = -1;  // residual value id (GEMM)
  // folded LayerNorm (bf16): the producer of a LayerNorm input writes its
  // row partials into value stats_out; the consumer GEMM reads them from
  // value ln_stats and applies the normalisation in its epilogue
  int stats_out = -1, stats_cols = 16, ln_stats = -1, ln_parts = 0, ln_cols = 16;
  const void *ln_cs = nullptr, *ln_bw = nullptr;
  float ln_eps = 0.f;
  // split-K GEMM: fp32 workspace value [splits, M, N] (live for this op only)
  int ws = -1, splits = 1;
};

// A LayerNorm folded into the Linear that consumes it (stats: the value that
// holds the input's row partials, each over `cols` columns; -1 = not
// folded, run the LayerNorm op).
struct LnFold {
  int stats = -1, d = 0, cols = 16;
  float eps = 0.f;
  std::string pfx;
  bool on() const { return stats >= 0; }
};

struct Param {
  std::vector<uint8_t> host;
  int dt = F32;
  Shape shape;  // informational
};

}  // namespace

struct EngineImpl {
  json::Value cfg;
  int device = 0;
  bool plan_only = false;
  int dt = F32;
  std::map<std::string, Param> params;
  // Instances compiled for further input shapes read the primary instance's
  // parameters and weight arena (the packed weights do not depend on the
  // input shape): pp points at the owning map, shared_wbuf at its arena.
  const std::map<std::string, Param> *pp = &params;
  std::set<std::string> used_params;  // names the lowering read
  char *shared_wbuf = nullptr;
  size_t shared_wbytes = 0;
  // pinned host staging for the PCIe path (allocated on first use)
  void *pin_in = nullptr, *pin_out = nullptr;
  // attention with textbook keys (DecoderLM "attention": "textbook")
  bool textbook_attn = false;
  // KV-cache prefill: every attention op also copies its k and v into the
  // caches of a decoder (attention layer i at kv_k / kv_v + i * kv_layer_bytes,
  // [B, H, kv_Lmax, hd] each); set before compile
  char *kv_k = nullptr, *kv_v = nullptr;
  size_t kv_layer_bytes = 0;
  int kv_Lmax = 0, attn_layers = 0;

  std::vector<Val> vals;
  std::vector<Op> ops;
  int input = -1, output = -1;
  bool stream_out = false;  // the final GEMM stores the output non-temporally
  bool prefetch = true;     // each GEMM touches the next GEMM's weights
  Shape in_shape;

  // device state
  hipStream_t stream = nullptr;
  char *arena = nullptr;
  size_t arena_bytes = 0;
  char *wbuf = nullptr;
  size_t wbytes = 0;
  std::vector<std::pair<std::vector<uint8_t>, size_t>> wpending;  // host bytes -> offset
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  bool compiled = false;

  // stats
  double compile_ms = 0, last_run_ms = 0, last_gpu_ms = 0, load_ms = 0;
  size_t runs = 0, fused_epilogues = 0, zero_copy_concats = 0, ln_folds = 0;

  ~EngineImpl() {
    if (plan_only) return;
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (arena) (void)hipFree(arena);
    if (wbuf && wbuf != shared_wbuf) (void)hipFree(wbuf);
    if (pin_in) (void)hipHostFree(pin_in);
    if (pin_out) (void)hipHostFree(pin_out);
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (stream) (void)hipStreamDestroy(stream);
  }

  // ---------------------------------------------------------------- values
  int new_val(const Shape &s, int vdt, int layout = ROWMAJOR) {
    Val v;
    v.shape = s;
    v.dt = vdt;
    v.layout = layout;
    vals.push_back(v);
    return int(vals.size()) - 1;
  }
  int alias(int base, const Shape &s, long off = 0, int layout = ROWMAJOR, long row_stride = 0) {
    int id = new_val(s, vals[base].dt, layout);
    vals[id].alias_of = base;
    vals[id].alias_off = off;
    vals[id].row_stride = row_stride;
    return id;
  }
  int root(int v) const {
    while (vals[v].alias_of >= 0) v = vals[v].alias_of;
    return v;
  }
  long elem_off(int v) const {
    long off = 0;
    while (vals[v].alias_of >= 0) {
      off += vals[v].alias_off;
      v = vals[v].alias_of;
    }
    return off;
  }
  Op &emit(int kind, const std::string &name, std::vector<int> in, std::vector<int> out) {
    Op o;
    o.kind = kind;
    o.name = name;
    o.in = std::move(in);
    o.out = std::move(out);
    ops.push_back(o);
    return ops.back();
  }

  // ---------------------------------------------------------------- params
  const Param &param(const std::string &n) {
    auto it = pp->find(n);
    if (it == pp->end()) throw Error("missing parameter '" + n + "'");
    if (it->second.dt != dt) throw Error("parameter '" + n + "' has the wrong dtype");
    used_params.insert(n);
    return it->second;
  }
  // A parameter that must hold exactly `count` elements of the engine dtype
  // (the reference's loader checks every shape, src/inference_serialization.cpp:
  // 863-881; LayerNorm its weight and bias, src/core/ops/normalization.cpp:141-145).
  const Param &param(const std::string &n, size_t count) {
    const Param &p = param(n);
    if (p.host.size() != count * dt_size(dt))
      throw Error("parameter '" + n + "' has " + std::to_string(p.host.size() / dt_size(dt)) + " elements, expected " +
                  std::to_string(count));
    return p;
  }
  // Pending device upload of host bytes into the weights arena.
  const void *upload(std::vector<uint8_t> bytes) {
    const size_t off = wbytes;
    wbytes += (bytes.size() + 255) & ~size_t(255);
    wpending.emplace_back(std::move(bytes), off);
    return reinterpret_cast<const void *>(off + 1);  // resolved after allocation (+1: never null)
  }
  // Linear weight [in, out] -> [out, in] (K-contiguous panels).
  // Linear weight [in, out] -> [out, in].  hwc (C, H, W): the input is a
  // flattened NHWC activation, its element (h W + w) C + c holding the
  // logical feature c H W + h W + w, so the K rows are permuted to match.
  std::vector<uint8_t> pack_linear(const Param &p, int in_f, int out_f, const int *hwc = nullptr) const {
    const size_t es = dt_size(dt);
    if (p.host.size() != size_t(in_f) * out_f * es) throw Error("linear weight has the wrong size");
    if (hwc && long(hwc[0]) * hwc[1] * hwc[2] != in_f) throw Error("linear weight: flattened input size mismatch");
    std::vector<uint8_t> t(p.host.size());
    for (int i = 0; i < in_f; ++i) {
      int src = i;
      if (hwc) {
        const int C = hwc[0], HW = hwc[1] * hwc[2], c = i % C, hw = i / C;
        src = c * HW + hw;
      }
      for (int o = 0; o < out_f; ++o)
        std::memcpy(&t[(size_t(o) * in_f + i) * es], &p.host[(size_t(src) * out_f + o) * es], es);
    }
    return t;
  }
  // Conv weight OIHW -> OHWI.
  // Conv weight [oC, iC, k, k] -> OHWI [oC, k, k, iCp], channels iC .. iCp-1
  // zero (iCp = iC unless the input layout is channel-padded).
  std::vector<uint8_t> pack_conv(const Param &p, int oC, int iC, int k, int iCp = 0) const {
    const size_t es = dt_size(dt);
    if (iCp < iC) iCp = iC;
    if (p.host.size() != size_t(oC) * iC * k * k * es) throw Error("conv weight has the wrong size");
    std::vector<uint8_t> t(size_t(oC) * k * k * iCp * es, 0);
    for (int o = 0; o < oC; ++o)
      for (int c = 0; c < iC; ++c)
        for (int q = 0; q < k * k; ++q)
          std::memcpy(&t[((size_t(o) * k * k + q) * iCp + c) * es], &p.host[((size_t(o) * iC + c) * k * k + q) * es], es);
    return t;
  }
  // ConvTranspose weight [iC, oC, k, k] -> [k, k, oC, iC].
  std::vector<uint8_t> pack_convt(const Param &p, int iC, int oC, int k) const {
    const size_t es = dt_size(dt);
    if (p.host.size() != size_t(oC) * iC * k * k * es) throw Error("conv_transpose weight has the wrong size");
    std::vector<uint8_t> t(p.host.size());
    for (int c = 0; c < iC; ++c)
      for (int o = 0; o < oC; ++o)
        for (int q = 0; q < k * k; ++q)
          std::memcpy(&t[((size_t(q) * oC + o) * iC + c) * es], &p.host[((size_t(c) * oC + o) * k * k + q) * es], es);
    return t;
  }
  const void *bias_or_zero(const std::string &n, int len) {
    if (pp->count(n)) return upload(param(n, size_t(len)).host);
    return upload(std::vector<uint8_t>(size_t(len) * dt_size(dt), 0));
  }

  // ---------------------------------------------------------------- lowering
  int to_rowmajor4(int x, const std::string &name) {
    if (vals[x].layout != NHWC) return x;
    // a 1x1 convolution to a few channels that produced x just now (the
    // output head) writes NCHW itself: x becomes the NCHW value
    if (!ops.empty()) {
      Op &pr = ops.back();
      if (pr.kind == OP_CONV && pr.out.size() == 1 && pr.out[0] == x && pr.a[9] == CONV_NHWC && pr.a[5] == 1 &&
          pr.a[6] == 1 && pr.a[7] == 0 && vals[x].alias_of < 0 && conv1x1_nchw_ok(dt, int(pr.a[1]), vals[pr.in[0]].row_stride ? vals[pr.in[0]].row_stride : pr.a[1], int(pr.a[4]))) {
        pr.a[9] = CONV_NCHW_OUT;
        vals[x].layout = ROWMAJOR;
        return x;
      }
    }
    const Shape s = vals[x].shape;
    int y = new_val(s, vals[x].dt, ROWMAJOR);
    Op &o = emit(OP_TO_NCHW, name + ".to_nchw", {x}, {y});
    o.a[0] = s[0]; o.a[1] = s[1]; o.a[2] = s[2] * s[3];
    return y;
  }
  // pad_to > C: the NHWC copy has pad_to channels, the extra ones zero (its
  // shape keeps the padded channel count; only a convolution reads it)
  int to_nhwc(int x, const std::string &name, int pad_to = 0) {
    if (vals[x].layout == NHWC) return x;
    Shape s = vals[x].shape;
    if (s.size() != 4) throw Error(name + ": expected a 4-D [B,C,H,W] input");
    const long C = s[1];
    if (pad_to > C) s[1] = pad_to;
    int y = new_val(s, vals[x].dt, NHWC);
    Op &o = emit(OP_TO_NHWC, name + ".to_nhwc", {x}, {y});
    o.a[0] = s[0]; o.a[1] = C; o.a[2] = s[2] * s[3]; o.a[3] = s[1];
    return y;
  }

  // LayerNorm(x) feeding a Linear, folded across the GEMM: possible when x
  // (bf16, row-major, d % 16 == 0) comes from a residual GEMM epilogue or the
  // embedding gather, which then also write x's row partials.  The consumer
  // multiplies the raw x by gamma (.) W and normalises in its epilogue:
  //   LN(x) W = rstd (x (gamma (.) W) - mean colsum(gamma (.) W)) + beta W.
  // (The reference rounds LN(x) to bf16 before its matmul; here the folded
  // weights are rounded instead, an error of the same order.)
  // consumer_n: the consuming Linear's output width.  Every column tile of
  // the consumer re-reads its rows' partials, so a consumer much wider than
  // d (a vocabulary head) keeps the LayerNorm kernel: measured on MI355X,
  // the 32000-wide LM head lost more than the LayerNorm launch costs.
  LnFold fold_ln(int x, const std::string &pfx, int d, float eps, long consumer_n) {
    LnFold f;
    const char *env = std::getenv("MUNET_HIP_LN_FOLD");  // "0" disables the fold (tests, comparisons)
    if ((env && env[0] == '0') || dt != BF16 || d % 16 || d > 1024 || consumer_n > 4L * d ||
        vals[x].layout != ROWMAJOR || vals[x].alias_of >= 0 || vals[x].shape.empty() || vals[x].shape.back() != d)
      return f;
    for (int i = int(ops.size()) - 1; i >= 0; --i) {
      Op &o = ops[i];
      if (std::find(o.out.begin(), o.out.end(), x) == o.out.end()) continue;
      // a GEMM writes the partials only from its bias + residual epilogue
      // program (no activation) on the pipelined kernel (K % 8 == 0); any
      // other producer keeps the LayerNorm kernel
      const bool gemm = o.kind == OP_GEMM && o.out[0] == x && o.a[1] == d && o.stats_out < 0 && o.b != nullptr &&
                        o.resid >= 0 && o.act == ACT_NONE && o.a[2] % 8 == 0;
      const bool embed = (o.kind == OP_EMBED || o.kind == OP_EMBED_POS) && o.out[0] == x && o.a[2] == d &&
                         o.stats_out < 0;
      if (!gemm && !embed) return f;
      // partial width: the embedding reduces whole rows; a GEMM producer
      // writes one partial per group of fragment columns that its wave
      // tiles cover whole (48 for the 128x96 tiles that N % 96 == 0 selects)
      f.cols = embed ? d : d % 96 == 0 ? 48 : d % 32 == 0 ? 32 : 16;
      const long M = long(numel(vals[x].shape) / d);
      f.stats = new_val({int(M), d / f.cols, 2}, F32);
      o.stats_out = f.stats;
      o.stats_cols = f.cols;
      o.out.push_back(f.stats);
      f.d = d;
      f.eps = eps;
      f.pfx = pfx;
      ++ln_folds;
      return f;
    }
    return f;
  }
  // Fold a LayerNorm's gamma into packed bf16 weights [out][in] and return
  // the epilogue terms: cs[o] = sum_k round(gamma_k w_ok), bw[o] = sum_k
  // beta_k w_ok (double sums).
  void fold_weights(std::vector<uint8_t> &packed, int in_f, int out_f, const LnFold &f, std::vector<uint8_t> &cs,
                    std::vector<uint8_t> &bw) {
    const Param &gp = param(f.pfx + "weight", size_t(in_f)), &bp = param(f.pfx + "bias", size_t(in_f));
    const uint16_t *gm = reinterpret_cast<const uint16_t *>(gp.host.data());
    const uint16_t *bt = reinterpret_cast<const uint16_t *>(bp.host.data());
    uint16_t *w = reinterpret_cast<uint16_t *>(packed.data());
    std::vector<float> csf(out_f), bwf(out_f);
    for (int o = 0; o < out_f; ++o) {
      double c = 0.0, b = 0.0;
      for (int k = 0; k < in_f; ++k) {
        uint16_t &wk = w[size_t(o) * in_f + k];
        const float wv = host_bf16_to_f32(wk);
        b += double(host_bf16_to_f32(bt[k])) * wv;
        wk = host_f32_to_bf16(host_bf16_to_f32(gm[k]) * wv);  // exact product, one rounding
        c += host_bf16_to_f32(wk);
      }
      csf[o] = float(c);
      bwf[o] = float(b);
    }
    cs.resize(size_t(out_f) * 4);
    bw.resize(size_t(out_f) * 4);
    std::memcpy(cs.data(), csf.data(), cs.size());
    std::memcpy(bw.data(), bwf.data(), bw.size());
  }
  void attach_fold(Op &o, const LnFold *ln, std::vector<uint8_t> &packed, int in_f, int out_f) {
    std::vector<uint8_t> cs, bw;
    fold_weights(packed, in_f, out_f, *ln, cs, bw);
    o.ln_stats = ln->stats;
    o.in.push_back(ln->stats);
    o.ln_cs = upload(std::move(cs));
    o.ln_bw = upload(std::move(bw));
    o.ln_parts = in_f / ln->cols;
    o.ln_cols = ln->cols;
    o.ln_eps = ln->eps;
  }

  // y = act(x W + b) (+ resid); x [..., in]; ln: a LayerNorm of x folded in
  int linear(int x, const std::string &pfx, int in_f, int out_f, bool has_bias, int act = ACT_NONE, int resid = -1,
             int out_val = -1, const LnFold *ln = nullptr, const int *hwc = nullptr) {
    x = to_rowmajor4(x, pfx);
    const Shape s = vals[x].shape;
    if (s.empty() || s.back() != in_f) throw Error(pfx + ": input " + shape_str(s) + " does not end in " + std::to_string(in_f));
    Shape os = s;
    os.back() = out_f;
    const int y = out_val >= 0 ? out_val : new_val(os, dt);
    Op &o = emit(OP_GEMM, pfx.empty() ? "linear" : pfx.substr(0, pfx.size() - 1), {x}, {y});
    o.a[0] = long(numel(s) / in_f);  // M
    o.a[1] = out_f;                  // N
    o.a[2] = in_f;                   // K
    std::vector<uint8_t> packed = pack_linear(param(pfx + "weight"), in_f, out_f, hwc);
    if (ln) {
      if (ln->d != in_f) throw Error(pfx + ": folded LayerNorm width mismatch");
      attach_fold(o, ln, packed, in_f, out_f);
    }
    o.w = upload(std::move(packed));
    o.b = has_bias ? bias_or_zero(pfx + "bias", out_f) : nullptr;
    o.act = act;
    if (resid >= 0) {
      o.resid = resid;
      o.in.push_back(resid);
    }
    if (act != ACT_NONE || resid >= 0) ++fused_epilogues;
    const int S = ln ? 1 : splitk_count(dt, int(o.a[0]), out_f, in_f);
    if (S > 1) {
      o.ws = new_val({S, int(o.a[0]), out_f}, F32);
      o.splits = S;
    }
    return y;
  }

  int conv(int x, const std::string &pfx, int iC, int oC, int k, int s, int p, int act, int out_view = -1) {
    // a 16-bit NCHW image of at most 3 channels into a 3x3 convolution: read
    // in place by the few-channel kernel (K = 9 C in one MFMA step), which
    // writes the NHWC activation; no converted copy of the image
    if (vals[x].layout != NHWC && vals[x].shape.size() == 4 && vals[x].shape[1] == iC &&
        conv3x3_fewc_ok(dt, iC, k, s, p, oC)) {
      const Shape xs = vals[x].shape;
      const int y = out_view >= 0 ? out_view : new_val({xs[0], oC, xs[2], xs[3]}, dt, NHWC);
      Op &o = emit(OP_CONV, pfx.substr(0, pfx.size() - 1), {x}, {y});
      o.a[0] = xs[0]; o.a[1] = iC; o.a[2] = xs[2]; o.a[3] = xs[3]; o.a[4] = oC; o.a[5] = k; o.a[6] = s; o.a[7] = p;
      o.a[8] = iC;
      o.a[9] = CONV_NCHW_IN;
      // OIHW rows (K = c 9 + kh 3 + kw) zero-padded to 32
      const Param &wp = param(pfx + "weight");
      const size_t es = dt_size(dt), row = size_t(iC) * 9 * es;
      if (wp.host.size() != size_t(oC) * row) throw Error(pfx + "weight has the wrong size");
      std::vector<uint8_t> w32(size_t(oC) * 32 * es, 0);
      for (int c = 0; c < oC; ++c) std::memcpy(&w32[size_t(c) * 32 * es], &wp.host[size_t(c) * row], row);
      o.w = upload(w32);
      o.b = bias_or_zero(pfx + "bias", oC);
      o.act = act;
      if (act != ACT_NONE) ++fused_epilogues;
      return y;
    }
    // an NCHW input with a channel count that is not a whole 16-byte chunk
    // (the image's 3 channels) converts to NHWC padded with zero channels, so
    // the convolution takes the vectorised im2col loader
    const int chunk = dt == F32 ? 4 : 8, padded = (iC + chunk - 1) / chunk * chunk;
    int iCp = iC;
    if (vals[x].layout == NHWC) {
      iCp = int(vals[x].shape[1]);  // an NHWC input may already carry the padding
      if (iCp != iC && iCp != padded) throw Error(pfx + ": channel mismatch");
    } else {
      if (vals[x].shape.size() == 4 && vals[x].shape[1] != iC) throw Error(pfx + ": channel mismatch");
      iCp = padded;
      x = to_nhwc(x, pfx, iCp);
    }
    const Shape xs = vals[x].shape;
    const int oH = (xs[2] + 2 * p - k) / s + 1, oW = (xs[3] + 2 * p - k) / s + 1;
    const int y = out_view >= 0 ? out_view : new_val({xs[0], oC, oH, oW}, dt, NHWC);
    Op &o = emit(OP_CONV, pfx.substr(0, pfx.size() - 1), {x}, {y});
    o.a[0] = xs[0]; o.a[1] = iCp; o.a[2] = xs[2]; o.a[3] = xs[3]; o.a[4] = oC; o.a[5] = k; o.a[6] = s; o.a[7] = p;
    o.a[8] = iC;  // the model's channels (the algorithmic work)
    o.w = upload(pack_conv(param(pfx + "weight"), oC, iC, k, iCp));
    o.b = bias_or_zero(pfx + "bias", oC);
    o.act = act;
    if (act != ACT_NONE) ++fused_epilogues;
    return y;
  }

  int unary(int x, int op, const std::string &name) {
    // fusion: fold ReLU / GELU into the producing GEMM / conv epilogue when
    // this op is its only consumer
    if (!ops.empty() && (op == UN_RELU || op == UN_GELU)) {
      Op &prev = ops.back();
      const bool producer = prev.out.size() == 1 && prev.out[0] == x;
      const bool gemm_ok = prev.kind == OP_GEMM && prev.resid < 0;
      const bool conv_ok = prev.kind == OP_CONV && op == UN_RELU;
      if (producer && (gemm_ok || conv_ok) && prev.act == ACT_NONE) {
        prev.act = op == UN_RELU ? ACT_RELU : ACT_GELU;
        prev.name += op == UN_RELU ? "+relu" : "+gelu";
        ++fused_epilogues;
        return x;
      }
    }
    int y = new_val(vals[x].shape, dt, vals[x].layout);
    Op &o = emit(OP_UNARY, name, {x}, {y});
    o.a[0] = op;
    o.a[1] = long(numel(vals[x].shape));
    o.f = host_round(dt, 1.702f);
    return y;
  }

  int layer_norm(int x, const std::string &pfx, int d, float eps) {
    x = to_rowmajor4(x, pfx);
    if (vals[x].shape.back() != d) throw Error(pfx + ": normalized_shape mismatch");
    int y = new_val(vals[x].shape, dt);
    Op &o = emit(OP_LN, pfx.substr(0, pfx.size() - 1), {x}, {y});
    o.a[0] = long(numel(vals[x].shape) / d);
    o.a[1] = d;
    o.f = eps;
    o.w = upload(param(pfx + "weight", size_t(d)).host);
    o.b = upload(param(pfx + "bias", size_t(d)).host);
    return y;
  }

  // nn::MultiHeadAttention (src/nn/attention.hpp:34-104) on x [B,T,E]; the
  // out-projection optionally adds a residual in its epilogue.
  int mha(int x, const std::string &pfx, int E, int H, bool causal, int resid = -1, const LnFold *ln = nullptr) {
    const Shape s = vals[x].shape;
    if (s.size() != 3 || s[2] != E) throw Error(pfx + ": MultiHeadAttention expects [B,T,E]");
    const int B = s[0], T = s[1], hd = E / H;
    if (E % H) throw Error(pfx + ": embed_dim must be divisible by num_heads");
    // the head-split epilogue stores 4 consecutive columns of one head
    if (hd % 4) throw Error(pfx + ": head_dim must be a multiple of 4 on the HIP engine");
    // fused q/k/v projection: weights [E,3E] -> [3E,E], biases [3E]
    std::vector<uint8_t> wcat, bcat;
    for (const char *p : {"q_proj.", "k_proj.", "v_proj."}) {
      auto w = pack_linear(param(pfx + p + "weight"), E, E);
      wcat.insert(wcat.end(), w.begin(), w.end());
      const auto &b = param(pfx + p + "bias", size_t(E)).host;
      bcat.insert(bcat.end(), b.begin(), b.end());
    }
    const int q = new_val({B * H, T, hd}, dt), k = new_val({B * H, T, hd}, dt), v = new_val({B * H, T, hd}, dt);
    Op &o = emit(OP_QKV, pfx + "qkv_proj", {x}, {q, k, v});
    o.a[0] = B; o.a[1] = T; o.a[2] = E; o.a[3] = H;
    if (ln) {
      if (ln->d != E) throw Error(pfx + ": folded LayerNorm width mismatch");
      attach_fold(o, ln, wcat, E, 3 * E);
    }
    o.w = upload(std::move(wcat));
    o.b = upload(std::move(bcat));
    const int ctx = new_val({B, T, E}, dt);
    Op &a = emit(OP_ATTN, pfx + "attention", {q, k, v}, {ctx});
    a.a[0] = B; a.a[1] = H; a.a[2] = T; a.a[3] = hd; a.a[4] = causal ? 1 : 0;
    a.a[5] = textbook_attn ? 1 : 0;
    a.a[6] = attn_layers++;
    a.f = host_round(dt, 1.0f / std::sqrt(float(hd)));
    return linear(ctx, pfx + "out_proj.", E, E, true, ACT_NONE, resid);
  }

  // Pre-LN transformer block: x + attn(ln1(x)), then x + ff(ln2(x))
  // (demos/multigpu/gpt3_multi_gpu_demo.py:105-114).
  // Both LayerNorms fold into the Linear that follows them when their input's
  // producer can write row partials (fold_ln).
  int block(int x, const std::string &pfx, int d, int H, int ffn, bool causal, float eps) {
    const LnFold f1 = fold_ln(x, pfx + "ln1.", d, eps, 3L * d);
    const int h = f1.on() ? x : layer_norm(x, pfx + "ln1.", d, eps);
    const int x2 = mha(h, pfx + "attn.", d, H, causal, x, f1.on() ? &f1 : nullptr);
    const LnFold f2 = fold_ln(x2, pfx + "ln2.", d, eps, ffn);
    const int h2 = f2.on() ? x2 : layer_norm(x2, pfx + "ln2.", d, eps);
    const int f = linear(h2, pfx + "ff.0.", d, ffn, true, ACT_GELU, -1, -1, f2.on() ? &f2 : nullptr);
    return linear(f, pfx + "ff.2.", ffn, d, true, ACT_NONE, x2);
  }

  int lower(const json::Value &m, int x, const std::string &pfx) {
    const std::string t = m.at("type").as_str();
    if (t == "Sequential") {
      const auto &layers = m.at("layers").arr;
      for (size_t i = 0; i < layers.size(); ++i) {
        // Flatten of a dense NHWC activation straight into a Linear: the
        // Linear reads the activation in place as [B, H W C] with its
        // weight's K rows permuted from the (C, H, W) order (no NCHW copy)
        const Val &xv = vals[x];
        if (i + 1 < layers.size() && layers[i].at("type").as_str() == "Flatten" &&
            layers[i + 1].at("type").as_str() == "Linear" && xv.layout == NHWC && xv.row_stride == 0 &&
            xv.shape.size() == 4) {
          const Shape xs = xv.shape;
          const int hwc[3] = {xs[1], xs[2], xs[3]};
          const int flat = alias(x, {xs[0], xs[1] * xs[2] * xs[3]});
          const json::Value &lin = layers[i + 1];
          x = linear(flat, pfx + std::to_string(i + 1) + ".", lin.at("in_features").as_int(),
                     lin.at("out_features").as_int(), lin.get_bool("bias", true), ACT_NONE, -1, -1, nullptr, hwc);
          ++i;
          continue;
        }
        x = lower(layers[i], x, pfx + std::to_string(i) + ".");
      }
      return x;
    }
    if (t == "Linear")
      return linear(x, pfx, m.at("in_features").as_int(), m.at("out_features").as_int(), m.get_bool("bias", true));
    if (t == "ReLU") return unary(x, UN_RELU, pfx + "relu");
    if (t == "Sigmoid") return unary(x, UN_SIGMOID, pfx + "sigmoid");
    if (t == "GELU") return unary(x, UN_GELU, pfx + "gelu");
    if (t == "Dropout" || t == "Identity") return x;  // eval mode
    if (t == "Softmax") {
      x = to_rowmajor4(x, pfx);
      int y = new_val(vals[x].shape, dt);
      Op &o = emit(OP_SOFTMAX, pfx + "softmax", {x}, {y});
      o.a[1] = vals[x].shape.back();
      o.a[0] = long(numel(vals[x].shape) / o.a[1]);
      return y;
    }
    if (t == "Conv2d")
      return conv(x, pfx, m.at("in_channels").as_int(), m.at("out_channels").as_int(), m.at("kernel_size").as_int(),
                  m.get_int("stride", 1), m.get_int("padding", 0), ACT_NONE);
    if (t == "MaxPool2d" || t == "Upsample") {
      const Shape xs = vals[x].shape;
      if (xs.size() != 4) throw Error(pfx + t + ": expected [B,C,H,W]");
      const bool pool = t == "MaxPool2d";
      const int k = pool ? m.at("kernel_size").as_int() : m.at("scale_factor").as_int();
      const int s = pool ? m.get_int("stride", k) : 1, p = pool ? m.get_int("padding", 0) : 0;
      Shape os = pool ? Shape{xs[0], xs[1], (xs[2] + 2 * p - k) / s + 1, (xs[3] + 2 * p - k) / s + 1}
                      : Shape{xs[0], xs[1], xs[2] * k, xs[3] * k};
      int y = new_val(os, dt, vals[x].layout);
      Op &o = emit(pool ? OP_POOL : OP_UPSAMPLE, pfx + (pool ? "max_pool2d" : "upsample2d"), {x}, {y});
      o.a[0] = xs[0]; o.a[1] = xs[1]; o.a[2] = xs[2]; o.a[3] = xs[3]; o.a[4] = k; o.a[5] = s; o.a[6] = p;
      o.a[7] = vals[x].layout == NHWC;
      return y;
    }
    if (t == "Flatten") {
      x = to_rowmajor4(x, pfx);
      const Shape xs = vals[x].shape;
      return alias(x, {xs[0], int(numel(xs) / xs[0])});
    }
    if (t == "LayerNorm") return layer_norm(x, pfx, m.at("normalized_shape").as_int(), float(m.get_num("eps", 1e-5)));
    if (t == "MultiHeadAttention")
      return mha(x, pfx, m.at("embed_dim").as_int(), m.at("num_heads").as_int(), m.get_bool("causal", true));
    if (t == "Embedding") {
      const Shape xs = vals[x].shape;
      const int V = m.at("num_embeddings").as_int(), D = m.at("embedding_dim").as_int();
      if (vals[x].dt != I32 || xs.size() != 2) throw Error(pfx + "Embedding: expects int32 [B,T] ids");
      int y = new_val({xs[0], xs[1], D}, dt);
      Op &o = emit(OP_EMBED, pfx + "embedding", {x}, {y});
      o.a[0] = long(numel(xs)); o.a[1] = V; o.a[2] = D; o.a[3] = 1;
      o.w = upload(param(pfx + "weight", size_t(V) * D).host);
      return y;
    }
    if (t == "TransformerBlock")
      return block(x, pfx, m.at("d_model").as_int(), m.at("num_heads").as_int(), m.at("ffn").as_int(),
                   m.get_bool("causal", false), float(m.get_num("eps", 1e-5)));
    if (t == "DecoderLM") {
      const Shape xs = vals[x].shape;
      const int V = m.at("vocab").as_int(), C = m.at("ctx").as_int(), d = m.at("d_model").as_int();
      const std::string attn = m.get_str("attention", "munet");
      if (attn != "munet" && attn != "textbook") throw Error("DecoderLM: attention must be \"munet\" or \"textbook\"");
      textbook_attn = attn == "textbook";
      if (vals[x].dt != I32 || xs.size() != 2) throw Error("DecoderLM: expects int32 [B,T] ids");
      if (xs[1] > C) throw Error("DecoderLM: sequence longer than the position table");
      // token + position gathers and their add, one rounding
      int h = new_val({xs[0], xs[1], d}, dt);
      Op &o = emit(OP_EMBED_POS, pfx + "embed", {x}, {h});
      o.a[0] = long(numel(xs)); o.a[1] = V; o.a[2] = d; o.a[3] = xs[1];
      o.w = upload(param(pfx + "token_embed.weight", size_t(V) * d).host);
      o.w2 = upload(param(pfx + "pos_embed.weight", size_t(C) * d).host);
      const int L = m.at("num_layers").as_int(), H = m.at("num_heads").as_int(), ffn = m.at("ffn").as_int();
      const float eps = float(m.get_num("eps", 1e-5));
      for (int i = 0; i < L; ++i) h = block(h, pfx + "blocks." + std::to_string(i) + ".", d, H, ffn, true, eps);
      const LnFold ff = fold_ln(h, pfx + "ln_f.", d, eps, V);
      if (!ff.on()) h = layer_norm(h, pfx + "ln_f.", d, eps);
      return linear(h, pfx + "head.", d, V, true, ACT_NONE, -1, -1, ff.on() ? &ff : nullptr);
    }
    if (t == "UNet") return unet(m, x, pfx);
    throw Error("unsupported module type '" + t + "'");
  }

  // Build-defined UNet (the reference has no transposed conv): per level two
  // conv3x3+ReLU and a stride-2 conv3x3+ReLU downsample; decoder levels
  // ConvTranspose2d(2,2) then cat([up, skip]) and two conv3x3+ReLU; 1x1 head.
  // The skip conv writes straight into the right half of its level's concat
  // buffer and the transposed conv into the left half (zero-copy concat).
  int unet(const json::Value &m, int x, const std::string &pfx) {
    std::vector<int> ch;
    for (const auto &c : m.at("channels").arr) ch.push_back(c.as_int());
    const int L = int(ch.size());
    int prev = m.at("in_channels").as_int();
    std::vector<int> cat(L, -1);
    for (int l = 0; l < L; ++l) {
      const int c = ch[l];
      x = conv(x, pfx + "enc" + std::to_string(l) + ".0.", prev, c, 3, 1, 1, ACT_RELU);
      if (l < L - 1) {
        const Shape xs = vals[x].shape;
        cat[l] = new_val({xs[0], 2 * c, xs[2], xs[3]}, dt, NHWC);
        const int skip = alias(cat[l], {xs[0], c, xs[2], xs[3]}, c, NHWC, 2 * c);
        x = conv(x, pfx + "enc" + std::to_string(l) + ".1.", c, c, 3, 1, 1, ACT_RELU, skip);
        ++zero_copy_concats;
        x = conv(x, pfx + "down" + std::to_string(l) + ".", c, c, 3, 2, 1, ACT_RELU);
      } else {
        x = conv(x, pfx + "enc" + std::to_string(l) + ".1.", c, c, 3, 1, 1, ACT_RELU);
      }
      prev = c;
    }
    for (int l = L - 2; l >= 0; --l) {
      const int c = ch[l];
      // the transposed-conv epilogue stores 4 consecutive output channels
      if (c % 4) throw Error(pfx + "up" + std::to_string(l) + ": channels must be a multiple of 4 on the HIP engine");
      const Shape xs = vals[x].shape;
      const int up = alias(cat[l], {xs[0], c, xs[2] * 2, xs[3] * 2}, 0, NHWC, 2 * c);
      Op &o = emit(OP_CONVT, pfx + "up" + std::to_string(l), {x}, {up});
      o.a[0] = xs[0]; o.a[1] = ch[l + 1]; o.a[2] = xs[2]; o.a[3] = xs[3]; o.a[4] = c; o.a[5] = 2;
      o.w = upload(pack_convt(param(pfx + "up" + std::to_string(l) + ".weight"), ch[l + 1], c, 2));
      o.b = bias_or_zero(pfx + "up" + std::to_string(l) + ".bias", c);
      x = conv(cat[l], pfx + "dec" + std::to_string(l) + ".0.", 2 * c, c, 3, 1, 1, ACT_RELU);
      x = conv(x, pfx + "dec" + std::to_string(l) + ".1.", c, c, 3, 1, 1, ACT_RELU);
    }
    return conv(x, pfx + "head.", ch[0], m.at("out_channels").as_int(), 1, 1, 0, ACT_NONE);
  }

  // ---------------------------------------------------------------- planner
  void plan() {
    const int n = int(vals.size());
    const int kUnset = 1 << 30;
    for (auto &v : vals) { v.def = kUnset; v.last = -2; }
    auto touch = [&](int v, int t) {
      const int r = root(v);
      vals[r].def = std::min(vals[r].def, t);
      vals[r].last = std::max(vals[r].last, t);
    };
    // the input buffer is live for the whole forward (and after it): callers
    // write it once through mh_engine_input_ptr and launch repeatedly, so no
    // later value may reuse its memory; the output lives until read
    touch(input, -1);
    for (int i = 0; i < int(ops.size()); ++i) {
      for (int v : ops[i].out) touch(v, i);
      for (int v : ops[i].in) touch(v, i);
      if (ops[i].ws >= 0) touch(ops[i].ws, i);
    }
    touch(input, int(ops.size()));
    touch(output, int(ops.size()));
    // roots ordered by size, placed at the lowest offset free for their interval
    std::vector<int> order;
    for (int v = 0; v < n; ++v)
      if (vals[v].alias_of < 0 && vals[v].last >= -1) order.push_back(v);
    std::sort(order.begin(), order.end(), [&](int a, int b) { return vals[a].bytes() > vals[b].bytes(); });
    std::vector<int> placed;
    arena_bytes = 0;
    for (int v : order) {
      const size_t sz = (vals[v].bytes() + 255) & ~size_t(255);
      std::vector<std::pair<long, long>> busy;
      for (int u : placed)
        if (!(vals[u].last < vals[v].def || vals[v].last < vals[u].def))
          busy.push_back({vals[u].offset, vals[u].offset + long((vals[u].bytes() + 255) & ~size_t(255))});
      std::sort(busy.begin(), busy.end());
      long off = 0;
      for (auto &b : busy) {
        if (off + long(sz) <= b.first) break;
        off = std::max(off, b.second);
      }
      vals[v].offset = off;
      arena_bytes = std::max(arena_bytes, size_t(off) + sz);
      placed.push_back(v);
    }
    for (int v = 0; v < n; ++v)
      if (vals[v].alias_of >= 0) vals[v].offset = vals[root(v)].offset + elem_off(v) * long(dt_size(vals[v].dt));
  }

  // ---------------------------------------------------------------- execution
  void *dptr(int v) const { return arena + vals[v].offset; }
  const void *wptr(const void *tag) const {
    return tag ? static_cast<const void *>(wbuf + (reinterpret_cast<uintptr_t>(tag) - 1)) : nullptr;
  }

  void set_fold(const Op &o, EpiArgs &ep) const {
    if (o.stats_out >= 0) {
      ep.stats_out = static_cast<float *>(dptr(o.stats_out));
      ep.stats_cols = o.stats_cols;
    }
    if (o.ln_stats >= 0) {
      ep.ln_stats = static_cast<const float *>(dptr(o.ln_stats));
      ep.ln_cs = static_cast<const float *>(wptr(o.ln_cs));
      ep.ln_bw = static_cast<const float *>(wptr(o.ln_bw));
      ep.ln_parts = o.ln_parts;
      ep.ln_cols = o.ln_cols;
      ep.ln_eps = o.ln_eps;
    }
  }

  // The weights of the first GEMM after op o, as o's GEMM prefetch target
  // (none past a convolution: its weights are read by other kernels).
  void set_prefetch(const Op &o, EpiArgs &ep) const {
    if (!prefetch || ops.empty() || &o < ops.data() || &o >= ops.data() + ops.size()) return;
    const long es = long(dt_size(dt));
    for (size_t i = size_t(&o - ops.data()) + 1; i < ops.size(); ++i) {
      const Op &n = ops[i];
      if (n.kind == OP_GEMM) {
        ep.pf = wptr(n.w);
        ep.pf_bytes = n.a[1] * n.a[2] * es;
        return;
      }
      if (n.kind == OP_QKV) {
        ep.pf = wptr(n.w);
        ep.pf_bytes = 3 * n.a[2] * n.a[2] * es;
        return;
      }
      if (n.kind == OP_CONV || n.kind == OP_CONVT) return;
    }
  }

  void enqueue(const Op &o) {
    hipStream_t st = stream;
    switch (o.kind) {
    case OP_GEMM: {
      EpiArgs ep;
      ep.out = dptr(o.out[0]);
      ep.ldc = o.a[1];
      ep.bias = wptr(o.b);
      ep.act = o.act;
      ep.gelu_c = host_round(dt, 1.702f);
      if (o.resid >= 0) {
        ep.resid = dptr(o.resid);
        ep.ldr = o.a[1];
      }
      set_fold(o, ep);
      set_prefetch(o, ep);
      ep.stream_out = o.out[0] == output && stream_out;
      if (o.splits > 1)
        hip_check(gemm_splitk(dt, dptr(o.in[0]), wptr(o.w), int(o.a[0]), int(o.a[1]), int(o.a[2]), o.splits,
                              static_cast<float *>(dptr(o.ws)), ep, st),
                  o.name.c_str());
      else
        hip_check(gemm_nt(dt, dptr(o.in[0]), wptr(o.w), int(o.a[0]), int(o.a[1]), int(o.a[2]), o.a[2], o.a[2], 1, 0,
                          0, 0, ep, -1, st),
                  o.name.c_str());
      break;
    }
    case OP_QKV: {
      const int B = int(o.a[0]), T = int(o.a[1]), E = int(o.a[2]), H = int(o.a[3]);
      EpiArgs ep;
      ep.mode = EPI_HEADSPLIT;
      ep.outs[0] = dptr(o.out[0]);
      ep.outs[1] = dptr(o.out[1]);
      ep.outs[2] = dptr(o.out[2]);
      ep.bias = wptr(o.b);
      ep.T = T; ep.H = H; ep.hd = E / H; ep.E = E;
      set_fold(o, ep);
      set_prefetch(o, ep);
      hip_check(gemm_nt(dt, dptr(o.in[0]), wptr(o.w), B * T, 3 * E, E, E, E, 1, 0, 0, 0, ep, -1, st), o.name.c_str());
      break;
    }
    case OP_ATTN:
      hip_check(attention(dt, dptr(o.in[0]), dptr(o.in[1]), dptr(o.in[2]), dptr(o.out[0]), int(o.a[0]), int(o.a[1]),
                          int(o.a[2]), int(o.a[3]), int(o.a[4]), o.f, 0, st, int(o.a[5])),
                o.name.c_str());
      if (kv_k)
        hip_check(kv_store(dt, dptr(o.in[1]), dptr(o.in[2]), kv_k + o.a[6] * kv_layer_bytes,
                           kv_v + o.a[6] * kv_layer_bytes, int(o.a[0] * o.a[1]), int(o.a[2]), int(o.a[3]), kv_Lmax, st),
                  (o.name + ".kv_store").c_str());
      break;
    case OP_LN:
      hip_check(layernorm(dt, dptr(o.in[0]), wptr(o.w), wptr(o.b), dptr(o.out[0]), int(o.a[0]), int(o.a[1]), o.f, st),
                o.name.c_str());
      break;
    case OP_EMBED:
    case OP_EMBED_POS:
      hip_check(embedding(dt, static_cast<const int32_t *>(dptr(o.in[0])), wptr(o.w),
                          o.kind == OP_EMBED_POS ? wptr(o.w2) : nullptr, dptr(o.out[0]), int(o.a[0]), int(o.a[1]),
                          int(o.a[2]), int(o.a[3]), device_error_flag(), st,
                          o.stats_out >= 0 ? static_cast<float *>(dptr(o.stats_out)) : nullptr),
                o.name.c_str());
      break;
    case OP_CONV: {
      if (o.a[9] == CONV_NCHW_IN) {
        EpiArgs ep;
        ep.out = dptr(o.out[0]);
        const Val &yo = vals[o.out[0]];
        ep.ldc = yo.row_stride ? yo.row_stride : o.a[4];
        ep.bias = wptr(o.b);
        ep.bias_first = 1;
        ep.act = o.act;
        hip_check(conv3x3_fewc(dt, dptr(o.in[0]), wptr(o.w), int(o.a[0]), int(o.a[1]), int(o.a[2]), int(o.a[3]),
                               int(o.a[4]), ep, st),
                  o.name.c_str());
        break;
      }
      if (o.a[9] == CONV_NCHW_OUT) {
        const Val &xi = vals[o.in[0]];
        const long M = o.a[0] * o.a[2] * o.a[3];
        hip_check(conv1x1_nchw(dt, dptr(o.in[0]), wptr(o.w), wptr(o.b), dptr(o.out[0]), M, int(o.a[2] * o.a[3]),
                               int(o.a[1]), xi.row_stride ? xi.row_stride : o.a[1], int(o.a[4]), o.act, st),
                  o.name.c_str());
        break;
      }
      ConvArgs cv;
      cv.B = int(o.a[0]); cv.iC = int(o.a[1]); cv.iH = int(o.a[2]); cv.iW = int(o.a[3]);
      cv.kH = cv.kW = int(o.a[5]); cv.s = int(o.a[6]); cv.p = int(o.a[7]);
      cv.oH = (cv.iH + 2 * cv.p - cv.kH) / cv.s + 1;
      cv.oW = (cv.iW + 2 * cv.p - cv.kW) / cv.s + 1;
      const Val &xi = vals[o.in[0]];
      cv.ldx = xi.row_stride ? xi.row_stride : cv.iC;
      const Val &yo = vals[o.out[0]];
      EpiArgs ep;
      ep.out = dptr(o.out[0]);
      ep.ldc = yo.row_stride ? yo.row_stride : o.a[4];
      ep.bias = wptr(o.b);
      ep.bias_first = 1;
      ep.act = o.act;
      hip_check(conv_nhwc(dt, dptr(o.in[0]), wptr(o.w), cv, int(o.a[4]), ep, -1, st), o.name.c_str());
      break;
    }
    case OP_CONVT: {
      const int B = int(o.a[0]), iC = int(o.a[1]), iH = int(o.a[2]), iW = int(o.a[3]), oC = int(o.a[4]),
                k = int(o.a[5]);
      const Val &yo = vals[o.out[0]];
      EpiArgs ep;
      ep.mode = EPI_CONVT;
      ep.out = dptr(o.out[0]);
      ep.ldc = yo.row_stride ? yo.row_stride : oC;
      ep.bias = wptr(o.b);
      ep.bias_first = 1;
      ep.convt_oc = oC; ep.convt_k = k; ep.convt_ih = iH; ep.convt_iw = iW;
      hip_check(gemm_nt(dt, dptr(o.in[0]), wptr(o.w), B * iH * iW, k * k * oC, iC, iC, iC, 1, 0, 0, 0, ep, -1, st),
                o.name.c_str());
      break;
    }
    case OP_POOL:
      hip_check(max_pool2d(dt, int(o.a[7]), dptr(o.in[0]), dptr(o.out[0]), int(o.a[0]), int(o.a[1]), int(o.a[2]),
                           int(o.a[3]), int(o.a[4]), int(o.a[5]), int(o.a[6]), st),
                o.name.c_str());
      break;
    case OP_UPSAMPLE:
      hip_check(upsample2d(dt, int(o.a[7]), dptr(o.in[0]), dptr(o.out[0]), int(o.a[0]), int(o.a[1]), int(o.a[2]),
                           int(o.a[3]), int(o.a[4]), st),
                o.name.c_str());
      break;
    case OP_UNARY:
      hip_check(mh::unary(dt, int(o.a[0]), dptr(o.in[0]), dptr(o.out[0]), size_t(o.a[1]), o.f, st), o.name.c_str());
      break;
    case OP_SOFTMAX:
      hip_check(softmax_rows(dt, dptr(o.in[0]), dptr(o.out[0]), int(o.a[0]), int(o.a[1]), st), o.name.c_str());
      break;
    case OP_TO_NHWC:
      if (o.a[3] > o.a[1])
        hip_check(nchw_to_nhwc_pad(vals[o.in[0]].dt, dptr(o.in[0]), dptr(o.out[0]), int(o.a[0]), int(o.a[1]),
                                   int(o.a[2]), int(o.a[3]), st),
                  o.name.c_str());
      else
        hip_check(nchw_to_nhwc(vals[o.in[0]].dt, dptr(o.in[0]), dptr(o.out[0]), int(o.a[0]), int(o.a[1]),
                               int(o.a[2]), st),
                  o.name.c_str());
      break;
    case OP_TO_NCHW:
      hip_check(nhwc_to_nchw(vals[o.in[0]].dt, dptr(o.in[0]), dptr(o.out[0]), int(o.a[0]), int(o.a[1]), int(o.a[2]), st),
                o.name.c_str());
      break;
    default:
      throw Error("engine: op kind not executable");
    }
  }

  void compile(const Shape &ishape) {
    const auto t0 = std::chrono::steady_clock::now();
    if (compiled) throw Error("engine already compiled");
    in_shape = ishape;
    vals.clear();
    ops.clear();
    attn_layers = 0;
    wbytes = 0;
    wpending.clear();
    const std::string t = cfg.at("type").as_str();
    const bool ids = t == "DecoderLM" || t == "Embedding";
    input = new_val(ishape, ids ? I32 : dt, ROWMAJOR);
    used_params.clear();
    int y = lower(cfg, input, "");
    // every parameter given must belong to the model (the reference's
    // load_state_dict rejects unknown names)
    for (const auto &kv : *pp)
      if (!used_params.count(kv.first)) throw Error("unknown parameter '" + kv.first + "' for this model");
    y = to_rowmajor4(y, "output");
    output = y;
    // a final output larger than the L2s and most of the last-level cache is
    // written with non-temporal stores (MUNET_HIP_STREAM_OUT=0 turns it off)
    const char *so = std::getenv("MUNET_HIP_STREAM_OUT");
    stream_out = vals[output].bytes() >= (size_t(64) << 20) && !(so && std::string(so) == "0");
    // the weights of a layer arrive cold from HBM (the forward's other
    // traffic evicts them between forwards): the GEMM before touches them
    // first (MUNET_HIP_PREFETCH=0 turns it off)
    const char *pfe = std::getenv("MUNET_HIP_PREFETCH");
    prefetch = !(pfe && std::string(pfe) == "0");
    plan();
    if (!plan_only) {
      hip_check(hipSetDevice(device), "hipSetDevice");
      hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
      hip_check(hipEventCreate(&ev0), "hipEventCreate");
      hip_check(hipEventCreate(&ev1), "hipEventCreate");
      hip_check(hipMalloc(&arena, std::max<size_t>(arena_bytes, 256)), "hipMalloc(arena)");
      if (shared_wbuf) {
        if (wbytes != shared_wbytes) throw Error("engine: weight layout differs between input shapes");
        wbuf = shared_wbuf;
      } else {
        hip_check(hipMalloc(&wbuf, std::max<size_t>(wbytes, 256)), "hipMalloc(weights)");
        for (auto &p : wpending)
          hip_check(hipMemcpy(wbuf + p.second, p.first.data(), p.first.size(), hipMemcpyHostToDevice),
                    "upload weights");
      }
      wpending.clear();
      wpending.shrink_to_fit();
      (void)device_error_flag();
      // zero the arena once so the warm-up reads defined memory
      hip_check(hipMemset(arena, 0, arena_bytes), "hipMemset(arena)");
      // warm-up eager forward (sets kernel attributes outside capture)
      for (const Op &o : ops) enqueue(o);
      hip_check(hipStreamSynchronize(stream), "warm-up forward");
      hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      try {
        for (const Op &o : ops) enqueue(o);
      } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      hip_check(hipStreamEndCapture(stream, &graph), "hipStreamEndCapture");
      hip_check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    }
    compiled = true;
    compile_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }

  void require_device() const {
    if (!compiled) throw Error("engine is not compiled");
    if (plan_only) throw Error("plan-only engine cannot run");
  }

  void launch() {
    require_device();
    hip_check(hipGraphLaunch(exec, stream), "hipGraphLaunch");
  }

  void run_device() {
    require_device();
    hip_check(hipEventRecord(ev0, stream), "hipEventRecord");
    hip_check(hipGraphLaunch(exec, stream), "hipGraphLaunch");
    hip_check(hipEventRecord(ev1, stream), "hipEventRecord");
    hip_check(hipStreamSynchronize(stream), "forward");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, ev0, ev1), "hipEventElapsedTime");
    last_gpu_ms = ms;
    set_last_kernel_time_us(double(ms) * 1000.0);
    ++runs;
  }

  // Algorithmic work of one op: FLOPs of its products (GEMM 2 M N K,
  // attention 4 B H T^2 hd, halved when causal, convolution 2 (B oH oW) oC
  // (k k iC), transposed convolution 2 (B iH iW k k) oC iC) and the unique bytes a
  // memory-bound op reads and writes (LayerNorm 2 M d s + 2 d s, embedding
  // 3 M d s + 4 M).
  void op_work(const Op &o, double &flops, double &bytes) const {
    const double es = double(dt_size(dt));
    flops = bytes = 0.0;
    switch (o.kind) {
    case OP_GEMM: flops = 2.0 * o.a[0] * o.a[1] * o.a[2]; break;
    case OP_QKV: flops = 2.0 * o.a[0] * o.a[1] * 3.0 * o.a[2] * o.a[2]; break;
    case OP_ATTN: flops = 4.0 * o.a[0] * o.a[1] * double(o.a[2]) * o.a[2] * o.a[3] * (o.a[4] ? 0.5 : 1.0); break;
    case OP_CONV: {  // 2 (B oH oW) oC (k k iC)
      const double oH = double((o.a[2] + 2 * o.a[7] - o.a[5]) / o.a[6] + 1),
                   oW = double((o.a[3] + 2 * o.a[7] - o.a[5]) / o.a[6] + 1);
      flops = 2.0 * o.a[0] * oH * oW * o.a[4] * double(o.a[5]) * o.a[5] * o.a[8];
      break;
    }
    case OP_CONVT: flops = 2.0 * o.a[0] * o.a[2] * o.a[3] * double(o.a[5]) * o.a[5] * o.a[4] * o.a[1]; break;
    case OP_LN: bytes = (2.0 * o.a[0] * o.a[1] + 2.0 * o.a[1]) * es; break;
    case OP_EMBED: case OP_EMBED_POS: bytes = 3.0 * o.a[0] * o.a[2] * es + 4.0 * o.a[0]; break;
    default: break;
    }
  }

  // GPU time of each op of the compiled forward on its own (the per-module
  // timings of the reference's Profiler, src/core/module.hpp:71-83, for the
  // compiled graph): before each op a full forward restores every value, then
  // `reps` launches of the op, captured in one graph on the engine stream, are
  // replayed once to warm and once between events.  An op never writes the
  // values it reads (the planner keeps them live through it), so its replays
  // recompute the same outputs.
  // only: time just the ops of that name (nullptr or "": every op).
  std::string op_times_json(int reps, const char *only) {
    require_device();
    if (reps < 1 || reps > 1000) throw Error("op_times: reps must be in 1..1000");
    std::ostringstream s;
    s << std::setprecision(15);
    s << "[";
    bool first = true;
    for (size_t i = 0; i < ops.size(); ++i) {
      if (only && *only && ops[i].name != only) continue;
      hip_check(hipGraphLaunch(exec, stream), "hipGraphLaunch");
      hipGraph_t g = nullptr;
      hipGraphExec_t x = nullptr;
      hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      try {
        for (int r = 0; r < reps; ++r) enqueue(ops[i]);
      } catch (...) {
        (void)hipStreamEndCapture(stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      hip_check(hipStreamEndCapture(stream, &g), "hipStreamEndCapture");
      float ms = 0.f;
      hipError_t err = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
      if (err == hipSuccess) err = hipGraphLaunch(x, stream);
      if (err == hipSuccess) err = hipEventRecord(ev0, stream);
      if (err == hipSuccess) err = hipGraphLaunch(x, stream);
      if (err == hipSuccess) err = hipEventRecord(ev1, stream);
      if (err == hipSuccess) err = hipStreamSynchronize(stream);
      if (err == hipSuccess) err = hipEventElapsedTime(&ms, ev0, ev1);
      if (x) (void)hipGraphExecDestroy(x);
      (void)hipGraphDestroy(g);
      hip_check(err, "op_times replay");
      double flops, bytes;
      op_work(ops[i], flops, bytes);
      s << (first ? "" : ",") << "{\"name\":\"" << ops[i].name << "\",\"kind\":\"" << op_name(ops[i].kind)
        << "\",\"us\":" << double(ms) * 1000.0 / reps << ",\"flops\":" << flops << ",\"bytes\":" << bytes << "}";
      first = false;
    }
    s << "]";
    hip_check(hipStreamSynchronize(stream), "op_times");
    return s.str();
  }

  // GPU time of each op inside the forward, with the caches and transitions
  // of the graph: for every prefix ops[0..i] of the forward, a graph of that
  // prefix is launched once to warm and then `reps` times back to back
  // between events; op i's time is T(i) - T(i-1).  Events inside a graph or
  // between eager launches would add their own packets (about 3 us per op);
  // differences of whole-graph times add nothing.  Op 0's time also holds
  // the graph launch overhead.
  std::string forward_op_times_json(int reps) {
    require_device();
    if (reps < 1 || reps > 1000) throw Error("forward_op_times: reps must be in 1..1000");
    const size_t n = ops.size();
    std::vector<double> prefix_ms(n, 0.0);
    for (size_t i = 0; i < n; ++i) {
      hipGraph_t g = nullptr;
      hipGraphExec_t x = nullptr;
      hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      try {
        for (size_t j = 0; j <= i; ++j) enqueue(ops[j]);
      } catch (...) {
        (void)hipStreamEndCapture(stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      hip_check(hipStreamEndCapture(stream, &g), "hipStreamEndCapture");
      float ms = 0.f;
      hipError_t err = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
      if (err == hipSuccess) err = hipGraphLaunch(x, stream);
      if (err == hipSuccess) err = hipEventRecord(ev0, stream);
      for (int r = 0; r < reps && err == hipSuccess; ++r) err = hipGraphLaunch(x, stream);
      if (err == hipSuccess) err = hipEventRecord(ev1, stream);
      if (err == hipSuccess) err = hipStreamSynchronize(stream);
      if (err == hipSuccess) err = hipEventElapsedTime(&ms, ev0, ev1);
      if (x) (void)hipGraphExecDestroy(x);
      (void)hipGraphDestroy(g);
      hip_check(err, "forward_op_times");
      prefix_ms[i] = double(ms) / reps;
    }
    std::ostringstream s;
    s << std::setprecision(15) << "[";
    for (size_t i = 0; i < n; ++i) {
      double flops, bytes;
      op_work(ops[i], flops, bytes);
      const double us = (prefix_ms[i] - (i ? prefix_ms[i - 1] : 0.0)) * 1000.0;
      s << (i ? "," : "") << "{\"name\":\"" << ops[i].name << "\",\"kind\":\"" << op_name(ops[i].kind)
        << "\",\"us\":" << us << ",\"flops\":" << flops << ",\"bytes\":" << bytes << "}";
    }
    s << "]";
    return s.str();
  }

  void check_error_flag() {
    int flag = 0;
    hip_check(hipMemcpy(&flag, device_error_flag(), sizeof(int), hipMemcpyDeviceToHost), "error flag");
    if (flag) {
      hip_check(hipMemset(device_error_flag(), 0, sizeof(int)), "clear error flag");
      throw Error("Embedding index out of range");
    }
  }

  // Host input -> device (hin == nullptr: the input buffer already holds it).
  double last_prepare_ms = 0;
  void stage_input(const void *hin) {
    const auto t0 = std::chrono::steady_clock::now();
    if (hin) hip_check(hipMemcpyAsync(dptr(input), hin, vals[input].bytes(), hipMemcpyHostToDevice, stream), "input H2D");
    last_prepare_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }

  void run(const void *hin, void *hout) {
    require_device();
    const auto t0 = std::chrono::steady_clock::now();
    stage_input(hin);
    run_device();
    hip_check(hipMemcpyAsync(hout, dptr(output), vals[output].bytes(), hipMemcpyDeviceToHost, stream), "output D2H");
    hip_check(hipStreamSynchronize(stream), "output D2H");
    check_error_flag();
    last_run_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }

  // Pinned host staging buffers sized to the input and the output.
  void pinned(void **in, void **out) {
    require_device();
    if (!pin_in) hip_check(hipHostMalloc(&pin_in, std::max<size_t>(vals[input].bytes(), 64), hipHostMallocDefault), "hipHostMalloc(input)");
    if (!pin_out) hip_check(hipHostMalloc(&pin_out, std::max<size_t>(vals[output].bytes(), 64), hipHostMallocDefault), "hipHostMalloc(output)");
    *in = pin_in;
    *out = pin_out;
  }

  // Forward from the pinned input staging buffer into the pinned output one.
  void run_pinned() {
    void *pi, *po;
    pinned(&pi, &po);
    run(pi, po);
  }

  std::string stats_json() const {
    std::ostringstream s;
    s << "{\"runs\":" << runs << ",\"compile_ms\":" << compile_ms << ",\"last_run_ms\":" << last_run_ms
      << ",\"last_forward_gpu_ms\":" << last_gpu_ms << ",\"compiled_input_shape\":" << shape_str(in_shape)
      << ",\"compiled_output_shape\":" << (output >= 0 ? shape_str(vals[output].shape) : "[]")
      << ",\"arena_bytes\":" << arena_bytes << ",\"weight_bytes\":" << wbytes << ",\"ops\":" << ops.size()
      << ",\"fused_epilogues\":" << fused_epilogues << ",\"ln_folds\":" << ln_folds << ",\"stream_out\":" << (stream_out ? "true" : "false")
      << ",\"prefetch\":" << (prefetch ? "true" : "false")
      << ",\"zero_copy_concats\":" << zero_copy_concats
      << ",\"current_memory_bytes\":" << (arena_bytes + wbytes) << ",\"peak_memory_bytes\":" << (arena_bytes + wbytes)
      << "}";
    return s.str();
  }

  std::string plan_json() const {
    std::ostringstream s;
    s << "{\"arena_bytes\":" << arena_bytes << ",\"input\":" << input << ",\"output\":" << output << ",\"ops\":[";
    for (size_t i = 0; i < ops.size(); ++i) {
      const Op &o = ops[i];
      s << (i ? "," : "") << "{\"kind\":\"" << op_name(o.kind) << "\",\"name\":\"" << o.name << "\",\"act\":" << o.act
        << ",\"resid\":" << o.resid << ",\"stats_out\":" << o.stats_out << ",\"ln_stats\":" << o.ln_stats << ",\"in\":[";
      for (size_t j = 0; j < o.in.size(); ++j) s << (j ? "," : "") << o.in[j];
      s << "],\"out\":[";
      for (size_t j = 0; j < o.out.size(); ++j) s << (j ? "," : "") << o.out[j];
      s << "]}";
    }
    s << "],\"values\":[";
    for (size_t v = 0; v < vals.size(); ++v) {
      const Val &x = vals[v];
      s << (v ? "," : "") << "{\"shape\":" << shape_str(x.shape) << ",\"dtype\":" << x.dt << ",\"bytes\":" << x.bytes()
        << ",\"offset\":" << x.offset << ",\"alias_of\":" << x.alias_of << ",\"def\":" << vals[root(int(v))].def
        << ",\"last\":" << vals[root(int(v))].last << ",\"layout\":" << x.layout << "}";
    }
    s << "]}";
    return s.str();
  }
};

}  // namespace mh

// The engine handle: the primary compiled instance plus the caller-side
// features of the reference Engine (src/inference.hpp:31-41, 128-289,
// 446-627): an input shape contract with -1 wildcards served by one compiled
// instance per concrete shape, the prepared-input cache, batch runs, an
// observer and EngineStats.
struct mh_engine {
  mh::EngineImpl impl;  // primary instance: owns the config, parameters and weights

  // input shape contract (reference ShapeContract): empty = exact, else -1 wildcards
  std::vector<int> expected;
  std::map<std::vector<int>, std::unique_ptr<mh::EngineImpl>> shapes;  // further instances

  // prepared-input cache (reference PreparedInputCache): device copies of host
  // inputs keyed by the caller's tensor identity and version, FIFO eviction
  struct Prepared {
    uint64_t key = 0, version = 0;
    size_t bytes = 0;
    void *dev = nullptr;
  };
  std::vector<Prepared> cache;
  size_t cache_max_entries = 8, cache_max_bytes = size_t(64) << 20, cache_bytes = 0;
  size_t cache_hits = 0, cache_misses = 0, cache_evictions = 0;

  mh_engine_observer observer = nullptr;
  void *observer_user = nullptr;
  size_t runs = 0;
  double last_run_ms = 0, last_prepare_ms = 0, last_forward_ms = 0, last_validate_ms = 0;

  // EngineConfig (reference src/inference.hpp:32-41, setters :311-335)
  int warmup_runs = 0;              // compile runs warmup_runs - 1 forwards after the first
  bool strict_shape_check = true;   // false: any input shape gets its own instance
  bool lean_mode = false;           // no memory figures or parameter scan in events
  bool loaded = false;
  double compile_warmup_ms = 0;
  // trace ids (reference next_trace_id / should_enable_trace_contexts,
  // src/inference.hpp:720-722): a fresh id per compile and per run while an
  // observer is attached, 0 otherwise; events carry the current one
  uint64_t next_trace = 0, current_trace = 0, last_compile_trace = 0, last_run_trace = 0;
  uint64_t new_trace() { return observer ? ++next_trace : 0; }

  ~mh_engine() { clear_cache(); }

  // Engine::load (reference src/inference.hpp:393-444): the parameters given
  // so far are the module; LoadStarted / LoadCompleted, with the parameter
  // count unless in lean mode.  compile() loads first when the caller did
  // not.
  void load() {
    if (loaded) return;
    current_trace = 0;
    emit("LoadStarted", 0.0, {}, {}, "Loading module into inference engine");
    std::ostringstream m;
    m << "Module loaded on hip:" << impl.device;
    if (!lean_mode) {
      size_t bytes = 0;
      for (const auto &kv : impl.params) bytes += kv.second.host.size();
      m << " (" << impl.params.size() << " parameter tensors, " << bytes << " bytes)";
    }
    loaded = true;
    emit("LoadCompleted", 0.0, {}, {}, m.str());
  }

  // Engine::compile's warm-up: warmup_runs - 1 forwards after the compile's
  // own first one (reference src/inference.hpp:507-515).
  void warmup() {
    compile_warmup_ms = 0;
    if (impl.plan_only) return;
    for (int i = 1; i < warmup_runs; ++i) {
      impl.run_device();
      compile_warmup_ms += impl.last_gpu_ms;
    }
  }

  void clear_cache() {
    for (auto &c : cache)
      if (c.dev) (void)hipFree(c.dev);
    cache.clear();
    cache_bytes = 0;
  }

  std::string mismatch(const std::vector<int> &actual) const {
    const std::vector<int> want = expected.empty() ? std::vector<int>(impl.in_shape.begin(), impl.in_shape.end()) : expected;
    if (actual.size() != want.size()) return "rank mismatch";
    for (size_t i = 0; i < want.size(); ++i)
      if (want[i] != -1 && want[i] != actual[i]) return "dim mismatch at index " + std::to_string(i);
    return {};
  }

  // The instance compiled for `shape` (compiled on first use).
  mh::EngineImpl &instance(const std::vector<int> &shape) {
    if (!impl.compiled) throw mh::Error("engine is not compiled");
    if (std::vector<int>(impl.in_shape.begin(), impl.in_shape.end()) == shape) return impl;
    const std::string why = mismatch(shape);
    if (!why.empty() && strict_shape_check) throw mh::Error("Engine: input shape mismatch with compiled shape: " + why);
    auto it = shapes.find(shape);
    if (it != shapes.end()) return *it->second;
    auto inst = std::make_unique<mh::EngineImpl>();
    inst->cfg = impl.cfg;
    inst->dt = impl.dt;
    inst->device = impl.device;
    inst->plan_only = impl.plan_only;
    inst->pp = &impl.params;
    inst->shared_wbuf = impl.wbuf;
    inst->shared_wbytes = impl.wbytes;
    emit("CompileStarted", 0.0, shape, {}, "compiling an instance for a new input shape");
    inst->compile(mh::Shape(shape.begin(), shape.end()));
    const auto &os = inst->vals[inst->output].shape;
    emit("CompileCompleted", inst->compile_ms, shape, std::vector<int>(os.begin(), os.end()), "instance compiled");
    return *(shapes[shape] = std::move(inst));
  }

  static std::string json_str(const std::string &v) {
    std::string o = "\"";
    for (char c : v) {
      if (c == '"' || c == '\\') o += '\\';
      o += (c == '\n') ? ' ' : c;
    }
    return o + "\"";
  }
  static std::string json_shape(const std::vector<int> &s) {
    std::string o = "[";
    for (size_t i = 0; i < s.size(); ++i) o += (i ? "," : "") + std::to_string(s[i]);
    return o + "]";
  }
  size_t memory_bytes() const {
    size_t b = impl.arena_bytes + impl.wbytes + cache_bytes;
    for (const auto &kv : shapes) b += kv.second->arena_bytes;
    return b;
  }

  // Observer callback (reference EngineEvent, src/inference.hpp:68-94) as JSON.
  void emit(const char *type, double ms, const std::vector<int> &in, const std::vector<int> &out,
            const std::string &msg) const {
    if (!observer) return;
    std::ostringstream s;
    const size_t mem = lean_mode ? 0 : memory_bytes();
    s << "{\"type\":\"" << type << "\",\"device\":" << impl.device << ",\"trace_id\":" << current_trace
      << ",\"run_index\":" << runs << ",\"duration_ms\":" << ms << ",\"input_shape\":" << json_shape(in)
      << ",\"output_shape\":" << json_shape(out) << ",\"current_memory_bytes\":" << mem
      << ",\"peak_memory_bytes\":" << mem << ",\"message\":" << json_str(msg) << "}";
    observer(s.str().c_str(), observer_user);
  }

  // One forward on the instance for `shape`; `hin` host input (or nullptr when
  // `dev_in` holds a prepared device copy), `hout` host output.
  void run_one(const std::vector<int> &shape, const void *hin, const void *dev_in, void *hout) {
    const auto t0 = std::chrono::steady_clock::now();
    current_trace = last_run_trace = new_trace();
    mh::EngineImpl &e = instance(shape);
    e.require_device();
    const std::vector<int> os(e.vals[e.output].shape.begin(), e.vals[e.output].shape.end());
    emit("RunStarted", 0.0, shape, {}, "Starting inference run");
    try {
      const auto tp = std::chrono::steady_clock::now();
      if (dev_in)
        mh::hip_check(hipMemcpyAsync(e.dptr(e.input), dev_in, e.vals[e.input].bytes(), hipMemcpyDeviceToDevice, e.stream),
                      "prepared input D2D");
      else
        e.stage_input(hin);
      last_prepare_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - tp).count();
      e.run_device();
      last_forward_ms = e.last_gpu_ms;
      const auto tv = std::chrono::steady_clock::now();
      mh::hip_check(hipMemcpyAsync(hout, e.dptr(e.output), e.vals[e.output].bytes(), hipMemcpyDeviceToHost, e.stream),
                    "output D2H");
      mh::hip_check(hipStreamSynchronize(e.stream), "output D2H");
      e.check_error_flag();
      last_validate_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - tv).count();
    } catch (const std::exception &ex) {
      emit("Error", 0.0, shape, {}, std::string("run failed: ") + ex.what());
      throw;
    }
    ++runs;
    last_run_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    emit("RunCompleted", last_run_ms, shape, os, "Inference run completed");
  }

  // Reference Engine::prepare_input with the prepared-input cache
  // (src/inference.hpp:665-686, cache src/inference.hpp:186-289).
  const void *prepared(const void *hin, size_t bytes, uint64_t key, uint64_t version) {
    for (const auto &c : cache)
      if (c.key == key && c.version == version && c.bytes == bytes) {
        ++cache_hits;
        return c.dev;
      }
    ++cache_misses;
    if (cache_max_entries == 0 || cache_max_bytes == 0 || bytes > cache_max_bytes) return nullptr;
    for (auto it = cache.begin(); it != cache.end(); ++it)
      if (it->key == key) {  // same tensor, stale version: replace
        cache_bytes -= it->bytes;
        (void)hipFree(it->dev);
        cache.erase(it);
        break;
      }
    while (!cache.empty() && (cache.size() >= cache_max_entries || cache_bytes + bytes > cache_max_bytes)) {
      cache_bytes -= cache.front().bytes;
      (void)hipFree(cache.front().dev);
      cache.erase(cache.begin());
      ++cache_evictions;
    }
    Prepared c;
    c.key = key;
    c.version = version;
    c.bytes = bytes;
    mh::hip_check(hipMalloc(&c.dev, std::max<size_t>(bytes, 16)), "hipMalloc(prepared input)");
    mh::hip_check(hipMemcpy(c.dev, hin, bytes, hipMemcpyHostToDevice), "prepared input H2D");
    cache.push_back(c);
    cache_bytes += bytes;
    return cache.back().dev;
  }

  std::string stats_json() const {
    std::string s = impl.stats_json();
    // runs over every compiled instance (device-resident launches included)
    size_t total = impl.runs;
    for (const auto &kv : shapes) total += kv.second->runs;
    const std::string first = "{\"runs\":" + std::to_string(impl.runs);
    s = "{\"runs\":" + std::to_string(total) + s.substr(first.size());
    std::ostringstream x;
    x << ",\"host_runs\":" << runs << ",\"engine_last_run_ms\":" << last_run_ms
      << ",\"last_prepare_input_ms\":" << last_prepare_ms << ",\"last_forward_ms\":" << last_forward_ms
      << ",\"last_output_validation_ms\":" << last_validate_ms << ",\"compiled_instances\":" << (1 + shapes.size())
      << ",\"expected_input_shape\":" << json_shape(expected) << ",\"prepared_input_cache_entries\":" << cache.size()
      << ",\"prepared_input_cache_bytes\":" << cache_bytes << ",\"prepared_input_cache_hits\":" << cache_hits
      << ",\"prepared_input_cache_misses\":" << cache_misses
      << ",\"prepared_input_cache_evictions\":" << cache_evictions << ",\"engine_memory_bytes\":" << memory_bytes()
      << ",\"last_compile_trace_id\":" << last_compile_trace << ",\"last_run_trace_id\":" << last_run_trace
      << ",\"compile_warmup_ms\":" << compile_warmup_ms << ",\"warmup_runs\":" << warmup_runs
      << ",\"strict_shape_check\":" << (strict_shape_check ? "true" : "false")
      << ",\"lean_mode\":" << (lean_mode ? "true" : "false") << "}";
    // the primary instance's object minus its closing brace, then the engine's fields
    return s.substr(0, s.size() - 1) + x.str();
  }
};

// Greedy autoregressive decode with a KV cache over a compiled DecoderLM
// whose attention uses textbook keys (no counterpart in the reference; its
// attention's keys are not per position, see decode.hip).  The prefill is the
// engine's own forward for [B, T0] (one compiled instance per T0) with each
// attention op also storing its k and v into the caches; each decode step is
// one launch of a captured graph of weight-streaming kernels (decode.hip)
// that feeds B tokens at the device-resident position and writes the B
// greedy choices back as the next step's input (one graph per count of
// 256-key attention blocks, chosen by the host from the position it tracks).
struct mh_decoder {
  mh_engine *eng = nullptr;
  int dt = mh::BF16, B = 0, Lmax = 0, L = 0, d = 0, H = 0, hd = 0, ffn = 0, V = 0, C = 0, nsplit = 0;
  float eps = 1e-5f;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  char *wbuf = nullptr, *buf = nullptr, *cache = nullptr;
  size_t wbytes = 0, bufbytes = 0, cache_bytes = 0, layer_bytes = 0;
  struct LayerW {
    const void *ln1w, *ln1b, *wqkv, *bqkv, *wo, *bo, *ln2w, *ln2b, *w1, *b1, *w2, *b2;
  };
  std::vector<LayerW> lw;
  const void *tok = nullptr, *pos_tab = nullptr, *lnfw = nullptr, *lnfb = nullptr, *whead = nullptr, *bhead = nullptr;
  void *x = nullptr, *x1 = nullptr, *q = nullptr, *h = nullptr, *logits = nullptr;
  int32_t *ids = nullptr, *tokens = nullptr;
  int *state = nullptr;
  unsigned long long *best = nullptr;
  float *part_o = nullptr;
  float2 *part_ml = nullptr;
  // one step graph per count of active 256-key attention blocks (1..nsplit):
  // the step at position p runs graph p / 256 (its keys 0..p), so the
  // attention launches only blocks holding keys and the out-projection
  // combines only their shares (each of its blocks loads every head's
  // shares: the load count, not the bytes, sets its input stage's time)
  std::vector<hipGraph_t> graphs;
  std::vector<hipGraphExec_t> execs;
  std::map<int, std::unique_ptr<mh::EngineImpl>> prefills;  // by prompt length
  int pos = -1;  // host copy of state[0]; -1 before the first prefill
  double last_step_ms = 0, last_generate_ms = 0, last_prefill_ms = 0;
  size_t steps = 0;

  ~mh_decoder() {
    prefills.clear();
    for (hipGraphExec_t x : execs)
      if (x) (void)hipGraphExecDestroy(x);
    for (hipGraph_t g : graphs)
      if (g) (void)hipGraphDestroy(g);
    if (wbuf) (void)hipFree(wbuf);
    if (buf) (void)hipFree(buf);
    if (cache) (void)hipFree(cache);
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (stream) (void)hipStreamDestroy(stream);
  }

  void create(mh_engine *e, int batch, int max_len) {
    using mh::Error;
    using mh::hip_check;
    eng = e;
    mh::EngineImpl &pi = e->impl;
    if (!pi.compiled || pi.plan_only) throw Error("decoder: the engine must be compiled on a device first");
    const mh::json::Value &m = pi.cfg;
    if (m.at("type").as_str() != "DecoderLM") throw Error("decoder: the model must be a DecoderLM");
    if (m.get_str("attention", "munet") != "textbook")
      throw Error("decoder: the DecoderLM must use \"attention\": \"textbook\" (MuNet's attention has no per-position keys to cache)");
    dt = pi.dt;
    const size_t es = mh::dt_size(dt), ce = 16 / es;
    V = m.at("vocab").as_int(); C = m.at("ctx").as_int(); d = m.at("d_model").as_int();
    L = m.at("num_layers").as_int(); H = m.at("num_heads").as_int(); ffn = m.at("ffn").as_int();
    eps = float(m.get_num("eps", 1e-5));
    hd = d / H;
    if (batch < 1 || batch > 16) throw Error("decoder: batch must be in 1..16");
    if (max_len < 1 || max_len > C) throw Error("decoder: max_len must be in 1..ctx");
    if (max_len > 4096) throw Error("decoder: max_len above 4096 (16 attention blocks of 256 keys)");
    if (d % H || hd > 64 || hd % 8 || hd % int(ce) || d % int(ce) || ffn % int(ce))
      throw Error("decoder: d_model, ffn and head_dim must be multiples of 16 bytes, head_dim a multiple of 8 and <= 64");
    if (size_t(batch) * std::max(d, ffn) * es > 65536) throw Error("decoder: batch x width exceeds the 64 KiB row stage");
    B = batch;
    Lmax = max_len;
    nsplit = (Lmax + mh::kDecKeyBlock - 1) / mh::kDecKeyBlock;

    // weights, packed as the decode kernels read them ([out, in] rows)
    mh::EngineImpl pk;
    pk.plan_only = true;
    pk.pp = &pi.params;
    pk.dt = dt;
    std::vector<std::pair<std::vector<uint8_t>, const void **>> up;
    auto add = [&](std::vector<uint8_t> b, const void **dst) { up.emplace_back(std::move(b), dst); };
    auto vec = [&](const std::string &n, size_t cnt) { return pk.param(n, cnt).host; };
    auto bias = [&](const std::string &n, size_t cnt) {
      return pi.params.count(n) ? vec(n, cnt) : std::vector<uint8_t>(cnt * es, 0);
    };
    lw.resize(L);
    for (int i = 0; i < L; ++i) {
      const std::string p = "blocks." + std::to_string(i) + ".";
      LayerW &w = lw[i];
      add(vec(p + "ln1.weight", d), &w.ln1w);
      add(vec(p + "ln1.bias", d), &w.ln1b);
      std::vector<uint8_t> wq, bq;
      for (const char *n : {"q_proj.", "k_proj.", "v_proj."}) {
        auto t = pk.pack_linear(pk.param(p + "attn." + n + "weight"), d, d);
        wq.insert(wq.end(), t.begin(), t.end());
        auto b = vec(p + "attn." + n + "bias", d);
        bq.insert(bq.end(), b.begin(), b.end());
      }
      add(std::move(wq), &w.wqkv);
      add(std::move(bq), &w.bqkv);
      add(pk.pack_linear(pk.param(p + "attn.out_proj.weight"), d, d), &w.wo);
      add(vec(p + "attn.out_proj.bias", d), &w.bo);
      add(vec(p + "ln2.weight", d), &w.ln2w);
      add(vec(p + "ln2.bias", d), &w.ln2b);
      add(pk.pack_linear(pk.param(p + "ff.0.weight"), d, ffn), &w.w1);
      add(bias(p + "ff.0.bias", ffn), &w.b1);
      add(pk.pack_linear(pk.param(p + "ff.2.weight"), ffn, d), &w.w2);
      add(bias(p + "ff.2.bias", d), &w.b2);
    }
    add(vec("token_embed.weight", size_t(V) * d), &tok);
    add(vec("pos_embed.weight", size_t(C) * d), &pos_tab);
    add(vec("ln_f.weight", d), &lnfw);
    add(vec("ln_f.bias", d), &lnfb);
    add(pk.pack_linear(pk.param("head.weight"), d, V), &whead);
    add(bias("head.bias", V), &bhead);
    std::vector<size_t> offs;
    for (auto &u : up) {
      offs.push_back(wbytes);
      wbytes += (u.first.size() + 255) & ~size_t(255);
    }
    hip_check(hipSetDevice(pi.device), "hipSetDevice");
    hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
    hip_check(hipEventCreate(&ev0), "hipEventCreate");
    hip_check(hipEventCreate(&ev1), "hipEventCreate");
    hip_check(hipMalloc(&wbuf, wbytes), "hipMalloc(decoder weights)");
    for (size_t i = 0; i < up.size(); ++i) {
      hip_check(hipMemcpy(wbuf + offs[i], up[i].first.data(), up[i].first.size(), hipMemcpyHostToDevice),
                "upload decoder weights");
      *up[i].second = wbuf + offs[i];
    }

    // activations, scratch and the caches ([layer][b][h][Lmax][hd], K then V)
    size_t off = 0;
    auto carve = [&](size_t bytes) { const size_t o = off; off += (bytes + 255) & ~size_t(255); return o; };
    const size_t o_x = carve(size_t(B) * d * es), o_x1 = carve(size_t(B) * d * es), o_q = carve(size_t(B) * d * es),
                 o_h = carve(size_t(B) * ffn * es), o_lg = carve(size_t(B) * V * es), o_ids = carve(size_t(B) * 4),
                 o_tok = carve(size_t(Lmax) * B * 4), o_st = carve(16), o_best = carve(size_t(B) * 8),
                 o_ml = carve(size_t(B) * H * nsplit * 8), o_part = carve(size_t(B) * H * nsplit * hd * 4);
    bufbytes = off;
    hip_check(hipMalloc(&buf, bufbytes), "hipMalloc(decoder buffers)");
    hip_check(hipMemset(buf, 0, bufbytes), "hipMemset(decoder buffers)");
    x = buf + o_x; x1 = buf + o_x1; q = buf + o_q; h = buf + o_h; logits = buf + o_lg;
    ids = reinterpret_cast<int32_t *>(buf + o_ids);
    tokens = reinterpret_cast<int32_t *>(buf + o_tok);
    state = reinterpret_cast<int *>(buf + o_st);
    best = reinterpret_cast<unsigned long long *>(buf + o_best);
    part_ml = reinterpret_cast<float2 *>(buf + o_ml);
    part_o = reinterpret_cast<float *>(buf + o_part);
    layer_bytes = size_t(B) * H * Lmax * hd * es;
    cache_bytes = 2 * size_t(L) * layer_bytes;
    hip_check(hipMalloc(&cache, cache_bytes), "hipMalloc(KV cache)");
    hip_check(hipMemset(cache, 0, cache_bytes), "hipMemset(KV cache)");

    // the step graphs
    graphs.assign(size_t(nsplit), nullptr);
    execs.assign(size_t(nsplit), nullptr);
    for (int nb = 1; nb <= nsplit; ++nb) {
      hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      try {
        enqueue_step(nb);
      } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      hip_check(hipStreamEndCapture(stream, &graphs[nb - 1]), "hipStreamEndCapture");
      hip_check(hipGraphInstantiate(&execs[nb - 1], graphs[nb - 1], nullptr, nullptr, 0), "hipGraphInstantiate");
    }
  }

  // the step graph for the tokens fed at position p (keys 0..p)
  hipGraphExec_t exec_at(int p) const { return execs[size_t(std::min(nsplit, p / mh::kDecKeyBlock + 1) - 1)]; }

  char *kcache(int l) const { return cache + size_t(l) * layer_bytes; }
  char *vcache(int l) const { return cache + (size_t(L) + l) * layer_bytes; }

  // nb: attention blocks of 256 keys (those holding keys 0..pos)
  void enqueue_step(int nb) {
    using mh::hip_check;
    const float gelu_c = mh::host_round(dt, 1.702f), scale = mh::host_round(dt, 1.0f / std::sqrt(float(hd)));
    hip_check(mh::dec_embed(dt, ids, best, tokens, state, tok, pos_tab, x, B, V, d, Lmax, mh::device_error_flag(), stream),
              "decode embed");
    mh::DecLinear p;
    p.state = state; p.M = B; p.E = d; p.H = H; p.hd = hd; p.Lmax = Lmax; p.nsplit = nb; p.eps = eps;
    p.gelu_c = gelu_c;
    for (int l = 0; l < L; ++l) {
      const LayerW &w = lw[l];
      mh::DecLinear a = p;  // ln1 + q/k/v: q, and k / v into the caches at pos
      a.x = x; a.w = w.wqkv; a.bias = w.bqkv; a.ln_w = w.ln1w; a.ln_b = w.ln1b; a.out = q;
      a.kc = kcache(l); a.vc = vcache(l); a.N = 3 * d; a.K = d;
      hip_check(mh::dec_linear(dt, 0, a, stream), "decode ln1 + qkv");
      hip_check(mh::dec_attention(dt, q, kcache(l), vcache(l), state, part_o, part_ml, B, H, hd, Lmax, nb, scale, stream),
                "decode attention");
      mh::DecLinear o = p;  // attention shares -> out_proj + residual
      o.part_o = part_o; o.part_ml = part_ml; o.w = w.wo; o.bias = w.bo; o.resid = x; o.out = x1; o.N = d; o.K = d;
      hip_check(mh::dec_linear(dt, 4, o, stream), "decode out_proj");
      mh::DecLinear f = p;  // ln2 + ff.0 + GELU
      f.x = x1; f.w = w.w1; f.bias = w.b1; f.ln_w = w.ln2w; f.ln_b = w.ln2b; f.out = h; f.N = ffn; f.K = d;
      hip_check(mh::dec_linear(dt, 2, f, stream), "decode ln2 + ff.0 + gelu");
      mh::DecLinear g = p;  // ff.2 + residual
      g.x = h; g.w = w.w2; g.bias = w.b2; g.resid = x1; g.out = x; g.N = d; g.K = ffn;
      hip_check(mh::dec_linear(dt, 1, g, stream), "decode ff.2");
    }
    mh::DecLinear hd_ = p;  // ln_f + head, greedy choice folded into best
    hd_.x = x; hd_.w = whead; hd_.bias = bhead; hd_.ln_w = lnfw; hd_.ln_b = lnfb; hd_.out = logits; hd_.best = best;
    hd_.pending = state + 2; hd_.N = V; hd_.K = d;
    hip_check(mh::dec_linear(dt, 3, hd_, stream), "decode ln_f + head");
  }

  // the last step's pending choices fed back (the next step's first kernel
  // does it otherwise)
  void finish() {
    mh::hip_check(mh::dec_finish(best, ids, tokens, state, B, Lmax, stream), "decode finish");
  }

  // Prompt ids [B, T0] through the engine's forward (textbook attention), the
  // caches filled for positions 0..T0-1; logits_out [B, T0, V] optional.
  void prefill(const int32_t *hids, int T0, void *logits_out) {
    using mh::Error;
    using mh::hip_check;
    if (T0 < 1 || T0 > Lmax) throw Error("decoder: prompt length must be in 1..max_len");
    auto it = prefills.find(T0);
    if (it == prefills.end()) {
      auto inst = std::make_unique<mh::EngineImpl>();
      const mh::EngineImpl &pi = eng->impl;
      inst->cfg = pi.cfg;
      inst->dt = pi.dt;
      inst->device = pi.device;
      inst->pp = &pi.params;
      inst->shared_wbuf = pi.wbuf;
      inst->shared_wbytes = pi.wbytes;
      inst->kv_k = cache;
      inst->kv_v = cache + size_t(L) * layer_bytes;
      inst->kv_layer_bytes = layer_bytes;
      inst->kv_Lmax = Lmax;
      inst->compile(mh::Shape{B, T0});
      it = prefills.emplace(T0, std::move(inst)).first;
    }
    mh::EngineImpl &e = *it->second;
    const auto t0 = std::chrono::steady_clock::now();
    e.stage_input(hids);
    e.run_device();
    const size_t es = mh::dt_size(dt);
    const char *out = static_cast<const char *>(e.dptr(e.output));
    if (logits_out)
      hip_check(hipMemcpyAsync(logits_out, out, size_t(B) * T0 * V * es, hipMemcpyDeviceToHost, e.stream), "logits D2H");
    // the next input: each sequence's greedy choice at its last position
    for (int b = 0; b < B; ++b)
      hip_check(mh::argmax_rows(dt, out + (size_t(b) * T0 + T0 - 1) * V * es, ids + b, 1, V, e.stream), "prefill argmax");
    const int st[3] = {T0, 0, 0};
    hip_check(hipMemcpyAsync(state, st, sizeof(st), hipMemcpyHostToDevice, e.stream), "decoder state");
    hip_check(hipStreamSynchronize(e.stream), "prefill");
    e.check_error_flag();
    pos = T0;
    last_prefill_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }

  void require_room(int n) const {
    if (pos < 0) throw mh::Error("decoder: prefill first");
    if (pos + n > Lmax) throw mh::Error("decoder: position past max_len");
  }

  // One step at position pos: hids [B] (nullptr: the previous greedy
  // choice); logits_out [B, V] and next_ids [B] optional.
  void step(const int32_t *hids, void *logits_out, int32_t *next_ids) {
    using mh::hip_check;
    require_room(1);
    if (hids) hip_check(hipMemcpyAsync(ids, hids, size_t(B) * 4, hipMemcpyHostToDevice, stream), "decoder ids H2D");
    hip_check(hipEventRecord(ev0, stream), "hipEventRecord");
    hip_check(hipGraphLaunch(exec_at(pos), stream), "hipGraphLaunch");
    finish();
    hip_check(hipEventRecord(ev1, stream), "hipEventRecord");
    if (logits_out)
      hip_check(hipMemcpyAsync(logits_out, logits, size_t(B) * V * mh::dt_size(dt), hipMemcpyDeviceToHost, stream),
                "logits D2H");
    if (next_ids) hip_check(hipMemcpyAsync(next_ids, ids, size_t(B) * 4, hipMemcpyDeviceToHost, stream), "ids D2H");
    hip_check(hipStreamSynchronize(stream), "decode step");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, ev0, ev1), "hipEventElapsedTime");
    last_step_ms = ms;
    ++pos;
    ++steps;
    eng->impl.check_error_flag();
  }

  // n greedy steps back to back; tokens_out [n, B].
  void generate(int n, int32_t *tokens_out) {
    using mh::hip_check;
    if (n < 1) throw mh::Error("decoder: n must be positive");
    require_room(n);
    const int zero = 0;
    hip_check(hipMemcpyAsync(state + 1, &zero, sizeof(int), hipMemcpyHostToDevice, stream), "decoder state");
    hip_check(hipEventRecord(ev0, stream), "hipEventRecord");
    for (int i = 0; i < n; ++i) hip_check(hipGraphLaunch(exec_at(pos + i), stream), "hipGraphLaunch");
    finish();
    hip_check(hipEventRecord(ev1, stream), "hipEventRecord");
    if (tokens_out)
      hip_check(hipMemcpyAsync(tokens_out, tokens, size_t(n) * B * 4, hipMemcpyDeviceToHost, stream), "tokens D2H");
    hip_check(hipStreamSynchronize(stream), "generate");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, ev0, ev1), "hipEventElapsedTime");
    last_generate_ms = ms;
    pos += n;
    steps += size_t(n);
    eng->impl.check_error_flag();
  }

  std::string stats_json() const {
    std::ostringstream s;
    s << "{\"batch\":" << B << ",\"max_len\":" << Lmax << ",\"position\":" << pos << ",\"steps\":" << steps
      << ",\"weight_bytes\":" << wbytes << ",\"cache_bytes\":" << cache_bytes << ",\"buffer_bytes\":" << bufbytes
      << ",\"kernels_per_step\":" << (2 + 5 * L) << ",\"step_graphs\":" << nsplit << ",\"last_step_ms\":" << last_step_ms
      << ",\"last_generate_ms\":" << last_generate_ms << ",\"last_prefill_ms\":" << last_prefill_ms
      << ",\"prefill_instances\":" << prefills.size() << "}";
    return s.str();
  }
};

using mh::Error;

#define ENG_TRY(...)                   \
  try {                                \
    __VA_ARGS__;                       \
    return 0;                          \
  } catch (const std::exception &e) {  \
    mh::set_last_error(e.what());      \
    return 1;                          \
  }

static void put_str(const std::string &s, char *buf, size_t len) {
  if (!buf || !len) throw Error("null buffer");
  if (s.size() + 1 > len) throw Error("buffer too small: need " + std::to_string(s.size() + 1));
  std::memcpy(buf, s.c_str(), s.size() + 1);
}

extern "C" {

int mh_engine_create(mh_engine **e, const char *config_json, int device) {
  ENG_TRY({
    if (!e || !config_json) throw Error("null argument");
    auto eng = std::make_unique<mh_engine>();
    eng->impl.cfg = mh::json::parse(config_json);
    const std::string dts = eng->impl.cfg.get_str("dtype", "float32");
    if (dts == "float32") eng->impl.dt = mh::F32;
    else if (dts == "float16") eng->impl.dt = mh::F16;
    else if (dts == "bfloat16") eng->impl.dt = mh::BF16;
    else throw Error("unsupported dtype '" + dts + "'");
    eng->impl.device = device;
    eng->impl.plan_only = device < 0;
    *e = eng.release();
  })
}

int mh_engine_destroy(mh_engine *e) { ENG_TRY(delete e) }

int mh_engine_set_param(mh_engine *e, const char *name, const void *data, size_t bytes, int dtype) {
  ENG_TRY({
    if (!e || !name || (!data && bytes)) throw Error("null argument");
    if (e->impl.compiled) throw Error("parameters must be set before compile");
    mh::Param p;
    const int edt = e->impl.dt;
    const bool fl = dtype == mh::F32 || dtype == mh::F16 || dtype == mh::BF16;
    if (fl && dtype != edt) {
      // another floating dtype: convert to the engine's with MuNet's codecs,
      // as the reference's loader does with Tensor::to (src/tensor.cpp:249-284)
      const size_t ies = mh::dt_size(dtype), n = bytes / ies;
      if (n * ies != bytes) throw Error(std::string("parameter '") + name + "' has a ragged byte size");
      const uint8_t *src = static_cast<const uint8_t *>(data);
      p.host.resize(n * mh::dt_size(edt));
      for (size_t i = 0; i < n; ++i) {
        float v;
        if (dtype == mh::F32) std::memcpy(&v, src + 4 * i, 4);
        else {
          uint16_t h;
          std::memcpy(&h, src + 2 * i, 2);
          v = dtype == mh::F16 ? mh::host_f16_to_f32(h) : mh::host_bf16_to_f32(h);
        }
        if (edt == mh::F32) {
          std::memcpy(&p.host[4 * i], &v, 4);
        } else {
          const uint16_t h = edt == mh::F16 ? mh::host_f32_to_f16(v) : mh::host_f32_to_bf16(v);
          std::memcpy(&p.host[2 * i], &h, 2);
        }
      }
      p.dt = edt;
    } else {
      p.dt = dtype;
      p.host.assign(static_cast<const uint8_t *>(data), static_cast<const uint8_t *>(data) + bytes);
    }
    e->impl.params[name] = std::move(p);
  })
}

int mh_engine_compile(mh_engine *e, const int *shape, int ndim) {
  ENG_TRY({
    if (!e || !shape || ndim <= 0) throw Error("bad input shape");
    std::vector<int> ex(shape, shape + ndim);
    if (mh_engine_compile_expected(e, shape, ndim, ex.data()) != 0) throw Error(mh_last_error());
    e->expected.clear();  // exact contract
  })
}

int mh_engine_input_ptr(mh_engine *e, void **p) {
  ENG_TRY({
    e->impl.require_device();
    *p = e->impl.dptr(e->impl.input);
  })
}

int mh_engine_output_ptr(mh_engine *e, void **p) {
  ENG_TRY({
    e->impl.require_device();
    *p = e->impl.dptr(e->impl.output);
  })
}

int mh_engine_output_shape(mh_engine *e, int *shape, int *ndim) {
  ENG_TRY({
    if (!e->impl.compiled) throw Error("engine is not compiled");
    const auto &s = e->impl.vals[e->impl.output].shape;
    *ndim = int(s.size());
    for (size_t i = 0; i < s.size(); ++i) shape[i] = s[i];
  })
}

int mh_engine_run(mh_engine *e, const void *in, void *out) {
  ENG_TRY({
    if (!e->impl.compiled) throw Error("engine is not compiled");
    e->run_one(std::vector<int>(e->impl.in_shape.begin(), e->impl.in_shape.end()), in, nullptr, out);
  })
}

int mh_engine_compile_expected(mh_engine *e, const int *shape, int ndim, const int *expected) {
  ENG_TRY({
    if (!e || !shape || !expected || ndim <= 0) throw Error("bad input shape");
    for (int i = 0; i < ndim; ++i)
      if (expected[i] != -1 && expected[i] != shape[i])
        throw Error("Engine: compile expected_input_shape mismatch: dim mismatch at index " + std::to_string(i));
    e->load();
    const auto t0 = std::chrono::steady_clock::now();
    e->current_trace = e->last_compile_trace = e->new_trace();
    e->emit("CompileStarted", 0.0, std::vector<int>(shape, shape + ndim), {}, "Compiling inference shape contract");
    try {
      e->impl.compile(mh::Shape(shape, shape + ndim));
      e->warmup();
    } catch (const std::exception &ex) {
      e->emit("Error", 0.0, std::vector<int>(shape, shape + ndim), {}, std::string("compile failed: ") + ex.what());
      throw;
    }
    e->expected.assign(expected, expected + ndim);
    const auto &os = e->impl.vals[e->impl.output].shape;
    e->emit("CompileCompleted", std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count(),
            std::vector<int>(shape, shape + ndim), std::vector<int>(os.begin(), os.end()), "Inference compile completed");
  })
}

int mh_engine_output_shape_for(mh_engine *e, const int *shape, int ndim, int *out_shape, int *out_ndim) {
  ENG_TRY({
    if (!e || !shape || ndim <= 0 || !out_shape || !out_ndim) throw Error("bad argument");
    const mh::EngineImpl &inst = e->instance(std::vector<int>(shape, shape + ndim));
    const auto &s = inst.vals[inst.output].shape;
    *out_ndim = int(s.size());
    for (size_t i = 0; i < s.size(); ++i) out_shape[i] = s[i];
  })
}

int mh_engine_run_shaped(mh_engine *e, const void *in, const int *shape, int ndim, void *out) {
  ENG_TRY({
    if (!e || !shape || ndim <= 0) throw Error("bad input shape");
    e->run_one(std::vector<int>(shape, shape + ndim), in, nullptr, out);
  })
}

int mh_engine_run_cached(mh_engine *e, const void *in, uint64_t key, uint64_t version, void *out) {
  ENG_TRY({
    if (!e->impl.compiled) throw Error("engine is not compiled");
    e->impl.require_device();
    const void *dev = e->prepared(in, e->impl.vals[e->impl.input].bytes(), key, version);
    e->run_one(std::vector<int>(e->impl.in_shape.begin(), e->impl.in_shape.end()), in, dev, out);
  })
}

int mh_engine_run_batch(mh_engine *e, int n, const void *const *inputs, void *const *outputs) {
  ENG_TRY({
    if (n < 0 || (n > 0 && (!inputs || !outputs))) throw Error("bad batch");
    if (!e->impl.compiled) throw Error("engine is not compiled");
    const std::vector<int> shape(e->impl.in_shape.begin(), e->impl.in_shape.end());
    for (int i = 0; i < n; ++i) e->run_one(shape, inputs[i], nullptr, outputs[i]);
  })
}

int mh_engine_load(mh_engine *e) { ENG_TRY(e->load()) }

int mh_engine_set_config(mh_engine *e, int warmup_runs, int strict_shape_check, int lean_mode) {
  ENG_TRY({
    if (warmup_runs < 0) throw Error("Engine warmup_runs must be >= 0");
    e->warmup_runs = warmup_runs;
    e->strict_shape_check = strict_shape_check != 0;
    e->lean_mode = lean_mode != 0;
  })
}

int mh_engine_set_input_cache(mh_engine *e, size_t max_entries, size_t max_bytes) {
  ENG_TRY({
    e->cache_max_entries = max_entries;
    e->cache_max_bytes = max_bytes;
    e->clear_cache();
  })
}

int mh_engine_clear_input_cache(mh_engine *e) { ENG_TRY(e->clear_cache()) }

int mh_engine_set_observer(mh_engine *e, mh_engine_observer fn, void *user) {
  ENG_TRY({
    e->observer = fn;
    e->observer_user = user;
  })
}

int mh_engine_pinned_io(mh_engine *e, void **in, void **out) { ENG_TRY(e->impl.pinned(in, out)) }
int mh_engine_run_pinned(mh_engine *e) {
  ENG_TRY({
    void *pi, *po;
    e->impl.pinned(&pi, &po);
    e->run_one(std::vector<int>(e->impl.in_shape.begin(), e->impl.in_shape.end()), pi, nullptr, po);
  })
}
int mh_engine_run_device(mh_engine *e) { ENG_TRY(e->impl.run_device()) }
int mh_engine_launch(mh_engine *e) { ENG_TRY(e->impl.launch()) }
int mh_engine_stream(mh_engine *e, void **s) {
  ENG_TRY({
    e->impl.require_device();
    *s = e->impl.stream;
  })
}
int mh_engine_stats(mh_engine *e, char *buf, size_t len) { ENG_TRY(put_str(e->stats_json(), buf, len)) }
int mh_engine_plan(mh_engine *e, char *buf, size_t len) { ENG_TRY(put_str(e->impl.plan_json(), buf, len)) }

int mh_engine_op_times(mh_engine *e, int reps, const char *only, char *buf, size_t len) {
  ENG_TRY(put_str(e->impl.op_times_json(reps, only), buf, len))
}

int mh_engine_forward_op_times(mh_engine *e, int reps, char *buf, size_t len) {
  ENG_TRY(put_str(e->impl.forward_op_times_json(reps), buf, len))
}

// ---- KV-cache decode -----------------------------------------------------------
int mh_decoder_create(mh_decoder **d, mh_engine *e, int batch, int max_len) {
  if (!d || !e) {
    mh::set_last_error("null handle");
    return 1;
  }
  *d = nullptr;
  auto dec = std::make_unique<mh_decoder>();
  ENG_TRY(dec->create(e, batch, max_len); *d = dec.release())
}
int mh_decoder_destroy(mh_decoder *d) { ENG_TRY(delete d) }
int mh_decoder_prefill(mh_decoder *d, const int32_t *ids, int T0, void *logits_out) {
  ENG_TRY(if (!d || !ids) throw Error("null argument"); d->prefill(ids, T0, logits_out))
}
int mh_decoder_step(mh_decoder *d, const int32_t *ids, void *logits_out, int32_t *next_ids) {
  ENG_TRY(if (!d) throw Error("null handle"); d->step(ids, logits_out, next_ids))
}
int mh_decoder_generate(mh_decoder *d, int n, int32_t *tokens_out, float *gpu_ms) {
  ENG_TRY(if (!d) throw Error("null handle"); d->generate(n, tokens_out); if (gpu_ms) *gpu_ms = float(d->last_generate_ms))
}
int mh_decoder_position(mh_decoder *d, int *pos) { ENG_TRY(if (!d || !pos) throw Error("null argument"); *pos = d->pos) }
int mh_decoder_stats(mh_decoder *d, char *buf, size_t len) {
  ENG_TRY(if (!d) throw Error("null handle"); put_str(d->stats_json(), buf, len))
}


}  // extern "C"
