// Thin C-ABI driver over the REAL MuNet CPU code, compiled from the sources
// under /root/reference by oracle/Makefile into oracle/_ref/. Test
// infrastructure only: it lets the tests pin the restatement
// (munet_cpu_ref.cpp) and write golden fixtures. Nothing here is copied from
// the reference: each entry point builds reference Tensors / nn modules and
// calls the reference's own ops:
//   ref_matmul       -> Tensor::matmul          (src/core/ops/matmul.cpp:394)
//   ref_binary       -> operator+ - * /         (src/core/ops/add.cpp, elementwise.cpp)
//   ref_relu/sigmoid -> ops::relu / sigmoid     (src/core/ops/activations.cpp:26-64)
//   ref_gelu         -> nn::GELU                (src/nn/activations.hpp:31-38)
//   ref_softmax      -> Tensor::softmax(-1)     (src/core/ops/activations.cpp:189)
//   ref_layer_norm   -> nn::LayerNorm           (src/nn/normalization.hpp:8-37)
//   ref_linear       -> nn::Linear              (src/nn/linear.hpp:9-37)
//   ref_mha          -> nn::MultiHeadAttention  (src/nn/attention.hpp:8-110)
//   ref_embedding    -> nn::Embedding (gather)  (src/nn/linear.hpp:75-149)
//   ref_conv2d       -> nn::Conv2d              (src/nn/linear.hpp:39-64)
//   ref_max_pool2d   -> nn::MaxPool2d           (src/nn/pooling.hpp:28-35)
//   ref_upsample2d   -> nn::Upsample            (src/nn/pooling.hpp:37-42)
//   ref_concat       -> Tensor::cat             (src/core/ops/shape.cpp:8-48)
//   ref_masked_fill  -> Tensor::masked_fill     (src/core/ops/elementwise.cpp:8-53)
//   ref_load_check   -> inference::load_serialized (src/inference_serialization.cpp:902-1080)
//   ref_load_forward -> load_serialized, then Module::forward (src/core/module.hpp:71-83)
#include "core/grad_mode.hpp"
#include "inference.hpp"
#include "nn/activations.hpp"
#include "nn/attention.hpp"
#include "nn/linear.hpp"
#include "nn/normalization.hpp"
#include "nn/pooling.hpp"
#include "tensor.hpp"

#include <cstring>
#include <memory>
#include <string>
#include <vector>

using namespace munet;

namespace {

thread_local std::string g_err;

DataType to_dt(int code) {
  switch (code) {
  case 0: return DataType::Float32;
  case 1: return DataType::Float16;
  case 2: return DataType::BFloat16;
  case 3: return DataType::Int32;
  }
  throw std::runtime_error("bad dtype code");
}

Shape mk_shape(const int *s, int n) { return Shape(s, s + n); }

Tensor from_host(const void *data, const Shape &shape, DataType dt) {
  Tensor t(shape, Device{DeviceType::CPU, 0}, dt, false);
  std::memcpy(t.data(), data, t.bytes());
  return t;
}

void to_host(const Tensor &t, void *out) {
  Tensor c = t.contiguous();
  std::memcpy(out, c.data(), c.bytes());
}

void set_param(Tensor &p, const void *data) {
  std::memcpy(p.data(), data, p.bytes());
}

} // namespace

#define REF_GUARD(...)                                                        \
  try {                                                                        \
    NoGradGuard ng;                                                            \
    __VA_ARGS__;                                                                    \
    return 0;                                                                  \
  } catch (const std::exception &e) {                                          \
    g_err = e.what();                                                          \
    return 1;                                                                  \
  }

extern "C" {

const char *ref_last_error() { return g_err.c_str(); }

int ref_encode(int dt, const float *src, void *dst, size_t n) {
  REF_GUARD({
    Tensor f = from_host(src, Shape{int(n)}, DataType::Float32);
    to_host(f.to(to_dt(dt)), dst);
  })
}

int ref_decode(int dt, const void *src, float *dst, size_t n) {
  REF_GUARD({
    Tensor t = from_host(src, Shape{int(n)}, to_dt(dt));
    to_host(t.to(DataType::Float32), dst);
  })
}

int ref_matmul(int dt, const void *a, const int *as, int an, const void *b,
               const int *bs, int bn, void *out) {
  REF_GUARD({
    Tensor ta = from_host(a, mk_shape(as, an), to_dt(dt));
    Tensor tb = from_host(b, mk_shape(bs, bn), to_dt(dt));
    to_host(ta.matmul(tb), out);
  })
}

int ref_binary(int dt, int op, const void *a, const int *as, int an,
               const void *b, const int *bs, int bn, void *out) {
  REF_GUARD({
    Tensor ta = from_host(a, mk_shape(as, an), to_dt(dt));
    Tensor tb = from_host(b, mk_shape(bs, bn), to_dt(dt));
    Tensor r = op == 0 ? ta + tb : op == 1 ? ta - tb : op == 2 ? ta * tb : ta / tb;
    to_host(r, out);
  })
}

int ref_relu(int dt, const void *in, void *out, size_t n) {
  REF_GUARD(to_host(from_host(in, Shape{int(n)}, to_dt(dt)).relu(), out))
}

int ref_sigmoid(int dt, const void *in, void *out, size_t n) {
  REF_GUARD(to_host(from_host(in, Shape{int(n)}, to_dt(dt)).sigmoid(), out))
}

int ref_gelu(int dt, const void *in, void *out, size_t n) {
  REF_GUARD({
    nn::GELU g;
    to_host(g.forward(from_host(in, Shape{int(n)}, to_dt(dt))), out);
  })
}

int ref_softmax(int dt, const void *in, void *out, int rows, int cols) {
  REF_GUARD(to_host(from_host(in, Shape{rows, cols}, to_dt(dt)).softmax(-1), out))
}

int ref_layer_norm(int dt, const void *x, const void *w, const void *b,
                   void *out, int rows, int cols, float eps) {
  REF_GUARD({
    TensorOptions o;
    o.dtype = to_dt(dt);
    nn::LayerNorm ln(cols, eps, o);
    set_param(ln.weight, w);
    set_param(ln.bias, b);
    to_host(ln.forward(from_host(x, Shape{rows, cols}, to_dt(dt))), out);
  })
}

// x: [rows, in] (2-D) or [B, T, in] (3-D when b_dim > 0)
int ref_linear(int dt, const void *x, const int *xs, int xn, const void *w,
               const void *bias, int in_f, int out_f, void *out) {
  REF_GUARD({
    TensorOptions o;
    o.dtype = to_dt(dt);
    nn::Linear lin(in_f, out_f, bias != nullptr, o);
    set_param(lin.weight, w);
    if (bias) set_param(lin.bias, bias);
    to_host(lin.forward(from_host(x, mk_shape(xs, xn), to_dt(dt))), out);
  })
}

// x: [B, T, E]; weights [E, E] ([in, out]) and biases [E] for q, k, v, out.
int ref_mha(int dt, const void *x, int B, int T, int E, int H, int causal,
            const void *wq, const void *bq, const void *wk, const void *bk,
            const void *wv, const void *bv, const void *wo, const void *bo,
            void *out) {
  REF_GUARD({
    TensorOptions o;
    o.dtype = to_dt(dt);
    nn::MultiHeadAttention mha(E, H, causal != 0, o);
    auto lin = [](const std::shared_ptr<nn::Module> &m) { return std::dynamic_pointer_cast<nn::Linear>(m); };
    set_param(lin(mha.q_proj)->weight, wq); set_param(lin(mha.q_proj)->bias, bq);
    set_param(lin(mha.k_proj)->weight, wk); set_param(lin(mha.k_proj)->bias, bk);
    set_param(lin(mha.v_proj)->weight, wv); set_param(lin(mha.v_proj)->bias, bv);
    set_param(lin(mha.out_proj)->weight, wo); set_param(lin(mha.out_proj)->bias, bo);
    to_host(mha.forward(from_host(x, Shape{B, T, E}, to_dt(dt))), out);
  })
}

int ref_embedding(int dt, const int32_t *ids, int B, int T, const void *weight,
                  int V, int D, void *out) {
  REF_GUARD({
    TensorOptions o;
    o.dtype = to_dt(dt);
    nn::Embedding emb(V, D, o);
    set_param(emb.weight, weight);
    emb.weight.set_requires_grad(false);
    to_host(emb.forward(from_host(ids, Shape{B, T}, DataType::Int32)), out);
  })
}

int ref_conv2d(int dt, const void *in, const void *w, const void *bias,
               void *out, int B, int iC, int iH, int iW, int oC, int k, int s,
               int p) {
  REF_GUARD({
    TensorOptions o;
    o.dtype = to_dt(dt);
    nn::Conv2d conv(iC, oC, k, s, p, o);
    set_param(conv.weight, w);
    if (bias) {
      set_param(conv.bias, bias);
    } else {
      conv.bias.fill_(0.0f);
    }
    to_host(conv.forward(from_host(in, Shape{B, iC, iH, iW}, to_dt(dt))), out);
  })
}

int ref_max_pool2d(int dt, const void *in, void *out, int B, int C, int iH,
                   int iW, int k, int s, int p) {
  REF_GUARD({
    nn::MaxPool2d mp(k, s, p);
    to_host(mp.forward(from_host(in, Shape{B, C, iH, iW}, to_dt(dt))), out);
  })
}

int ref_upsample2d(int dt, const void *in, void *out, int B, int C, int iH,
                   int iW, int scale) {
  REF_GUARD({
    nn::Upsample up(scale);
    to_host(up.forward(from_host(in, Shape{B, C, iH, iW}, to_dt(dt))), out);
  })
}

int ref_concat(int dt, const void *const *inputs, const int *shapes, int count,
               int ndim, int dim, void *out) {
  REF_GUARD({
    std::vector<Tensor> ts;
    for (int j = 0; j < count; ++j)
      ts.push_back(from_host(inputs[j], mk_shape(shapes + j * ndim, ndim), to_dt(dt)));
    to_host(Tensor::cat(ts, dim), out);
  })
}

// mask: int32 [n] (any non-zero entry selects `value`); value is the double
// a ScalarValue carries (src/types.hpp:201-208), as the op receives it.
int ref_masked_fill(int dt, const void *x, const int32_t *mask, void *out,
                    size_t n, double value) {
  REF_GUARD({
    Tensor tx = from_host(x, Shape{int(n)}, to_dt(dt));
    Tensor tm = from_host(mask, Shape{int(n)}, DataType::Int32);
    ScalarValue v;
    v.dtype = DataType::Float32;
    v.value = value;
    to_host(tx.masked_fill(tm, v), out);
  })
}

// MuNet's own deploy-artifact loader on `path`: 0 if it accepts the file,
// 1 with the loader's message (ref_last_error) if it refuses it.
int ref_load_check(const char *path) {
  REF_GUARD((void)inference::load_serialized(path, Device{DeviceType::CPU, 0}))
}

// Loads `path` with MuNet's loader and runs the module's forward on the host
// input x (dtype dt, shape xs[xn]); the output's bytes go to out (at most
// out_bytes), its shape to out_shape / *out_ndim (at most 8 dims).
int ref_load_forward(const char *path, int dt, const void *x, const int *xs, int xn, void *out, size_t out_bytes,
                     int *out_shape, int *out_ndim) {
  REF_GUARD({
    auto m = inference::load_serialized(path, Device{DeviceType::CPU, 0});
    Tensor y = m->forward(from_host(x, mk_shape(xs, xn), to_dt(dt))).contiguous();
    if (y.bytes() > out_bytes) throw std::runtime_error("ref_load_forward: output buffer too small");
    if (y.shape().size() > 8) throw std::runtime_error("ref_load_forward: output rank above 8");
    *out_ndim = int(y.shape().size());
    for (size_t i = 0; i < y.shape().size(); ++i) out_shape[i] = int(y.shape()[i]);
    to_host(y, out);
  })
}

} // extern "C"
