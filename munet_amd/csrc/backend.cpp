// munet_hip::HipBackend: the capability-interface mirror (hip_backend.hpp)
// implemented over the C ABI (include/munet_hip.h).  Every call checks the
// status and throws std::runtime_error with the library's message, the
// error convention of the reference's backends.
#include "hip_backend.hpp"

#include <algorithm>
#include <stdexcept>

#include "../../include/munet_hip.h"

namespace munet_hip {

namespace {
void ok(int rc) {
  if (rc != 0) throw std::runtime_error(mh_last_error());
}
int code(DataType d) { return static_cast<int>(d); }
int dev(Device d) { return d.type == DeviceType::CPU ? MH_DEVICE_CPU : MH_DEVICE_HIP; }
}  // namespace

BroadcastInfo compute_broadcast(const Shape &as, const Strides &ast, const Shape &bs, const Strides &bst) {
  const int nd = int(std::max(as.size(), bs.size()));
  BroadcastInfo info;
  info.out_shape.assign(nd, 1);
  info.strides_a.assign(nd, 0);
  info.strides_b.assign(nd, 0);
  for (int i = 0; i < nd; ++i) {
    const int ia = int(as.size()) - 1 - i, ib = int(bs.size()) - 1 - i, o = nd - 1 - i;
    const int da = ia >= 0 ? as[ia] : 1, db = ib >= 0 ? bs[ib] : 1;
    if (da != db && da != 1 && db != 1) return info;  // can_broadcast = false
    info.out_shape[o] = std::max(da, db);
    info.strides_a[o] = ia >= 0 ? ((da == 1 && db != 1) ? 0 : ast[ia]) : 0;
    info.strides_b[o] = ib >= 0 ? ((db == 1 && da != 1) ? 0 : bst[ib]) : 0;
  }
  info.can_broadcast = true;
  return info;
}

HipBackend::HipBackend(int device_index, void *stream) : device_(device_index), stream_(stream) {
  ok(mh_init(device_index));
}

BackendSupport HipBackend::query_support(BackendFeature, DataType dtype, const Shape *) const {
  BackendSupport s;
  s.available = dtype == DataType::Float32 || dtype == DataType::Float16 || dtype == DataType::BFloat16;
  s.fallback_policy = BackendFallbackPolicy::ExplicitUnsupported;
  s.preferred_accumulation_dtype = DataType::Float32;
  return s;
}

void *HipBackend::allocate(size_t bytes) {
  void *p = nullptr;
  ok(mh_allocate(&p, bytes));
  return p;
}
void HipBackend::deallocate(void *ptr) { ok(mh_deallocate(ptr)); }
void HipBackend::memset(void *ptr, int value, size_t bytes) { ok(mh_memset(ptr, value, bytes, stream_)); }
void HipBackend::copy(const void *src, void *dst, size_t bytes, Device s, Device d) {
  ok(mh_copy(src, dst, bytes, dev(s), dev(d), stream_));
}
void HipBackend::synchronize() { ok(mh_synchronize(stream_)); }
double HipBackend::get_last_kernel_time_us() { return mh_get_last_kernel_time_us(); }
void HipBackend::to_contiguous(const Storage &src, Storage &dst, const Shape &shape, const Strides &strides,
                               size_t offset) {
  ok(mh_to_contiguous(code(src.dtype), src.data, dst.data, int(shape.size()), shape.data(), strides.data(),
                      int64_t(offset), stream_));
}

#define MH_BIN(fn)                                                                                              \
  void HipBackend::fn(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info) {            \
    if (!info.can_broadcast) throw std::runtime_error(#fn ": shape mismatch");                                  \
    ok(mh_##fn(code(a.dtype), a.data, b.data, out.data, int(info.out_shape.size()), info.out_shape.data(),      \
               info.strides_a.data(), info.strides_b.data(), stream_));                                         \
  }
MH_BIN(add)
MH_BIN(sub)
MH_BIN(mul)
MH_BIN(div)
#undef MH_BIN

#define MH_UN(fn) \
  void HipBackend::fn(const Storage &in, Storage &out, size_t n) { ok(mh_##fn(code(in.dtype), in.data, out.data, n, stream_)); }
MH_UN(relu)
MH_UN(sigmoid)
MH_UN(exp)
MH_UN(log)
MH_UN(sqrt)
MH_UN(rsqrt)
MH_UN(sin)
MH_UN(cos)
MH_UN(gelu)
#undef MH_UN

void HipBackend::softmax(const Storage &in, Storage &out, int batch, int classes) {
  ok(mh_softmax(code(in.dtype), in.data, out.data, batch, classes, stream_));
}
void HipBackend::matmul(const Storage &a, const Storage &b, Storage &out, int M, int K, int N, bool ta, bool tb) {
  ok(mh_matmul(code(a.dtype), a.data, b.data, out.data, M, K, N, ta, tb, stream_));
}
void HipBackend::batched_matmul(const Storage &a, const Storage &b, Storage &out, int batch, int M, int K, int N,
                                bool ta, bool tb, int64_t sa, int64_t sb, int64_t sc) {
  ok(mh_batched_matmul(code(a.dtype), a.data, b.data, out.data, batch, M, K, N, ta, tb, sa, sb, sc, stream_));
}
void HipBackend::concat(const std::vector<Storage *> &inputs, Storage &out, int dim, const std::vector<Shape> &shapes) {
  if (inputs.empty() || shapes.size() != inputs.size()) throw std::runtime_error("concat: bad inputs");
  std::vector<const void *> ptrs;
  std::vector<int> flat;
  for (size_t i = 0; i < inputs.size(); ++i) {
    ptrs.push_back(inputs[i]->data);
    flat.insert(flat.end(), shapes[i].begin(), shapes[i].end());
  }
  ok(mh_concat(code(out.dtype), ptrs.data(), int(ptrs.size()), out.data, dim, int(shapes[0].size()), flat.data(),
               stream_));
}
void HipBackend::conv2d(const Storage &in, const Storage &w, const Storage *bias, Storage &out, int B, int iC, int iH,
                        int iW, int oC, int kH, int kW, int s, int p) {
  ok(mh_conv2d(code(in.dtype), in.data, w.data, bias ? bias->data : nullptr, out.data, B, iC, iH, iW, oC, kH, kW, s,
               p, stream_));
}
void HipBackend::max_pool2d(const Storage &in, Storage &out, int B, int C, int iH, int iW, int k, int s, int p) {
  ok(mh_max_pool2d(code(in.dtype), in.data, out.data, B, C, iH, iW, k, s, p, stream_));
}
void HipBackend::upsample2d(const Storage &in, Storage &out, int B, int C, int iH, int iW, int scale) {
  ok(mh_upsample2d(code(in.dtype), in.data, out.data, B, C, iH, iW, scale, stream_));
}
void HipBackend::layer_norm(const Storage &x, const Storage &w, const Storage &b, Storage &out, int rows, int cols,
                            float eps) {
  ok(mh_layer_norm(code(x.dtype), x.data, w.data, b.data, out.data, rows, cols, eps, stream_));
}
void HipBackend::masked_fill(const Storage &x, const Storage &mask, Storage &out, size_t n, double value) {
  ok(mh_masked_fill(code(x.dtype), x.data, static_cast<const int32_t *>(mask.data), out.data, n, value, stream_));
}
void HipBackend::embedding(const Storage &ids, const Storage &w, Storage &out, int n, int V, int D) {
  ok(mh_embedding(code(w.dtype), static_cast<const int32_t *>(ids.data), w.data, out.data, n, V, D, stream_));
}
void HipBackend::attention(const Storage &q, const Storage &k, const Storage &v, Storage &ctx, int B, int H, int T,
                           int hd, bool causal) {
  ok(mh_attention(code(q.dtype), q.data, k.data, v.data, ctx.data, B, H, T, hd, causal, stream_));
}

}  // namespace munet_hip

// C entry used by tests to check the C++ mirror links and reports support.
extern "C" int mh_backend_selftest(void) {
  munet_hip::BroadcastInfo bi = munet_hip::compute_broadcast({2, 3}, {3, 1}, {3}, {1});
  return (bi.can_broadcast && bi.strides_b[0] == 0 && bi.out_shape[1] == 3) ? 0 : 1;
}
