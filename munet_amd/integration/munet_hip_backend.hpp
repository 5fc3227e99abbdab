// munet::HIPBackend: the Backend subclass a MuNet build registers for the HIP
// device (the file a maintainer adds as src/backend/hip_backend.hpp).  It
// implements every pure virtual of the capability interfaces it provides
// (reference src/core/backend.hpp:190-311): allocation/transfer, elementwise,
// blas, shape and spatial, each forwarding to the C ABI of libmunet_hip.so
// (include/munet_hip.h) with the operands' raw storage pointers and dtypes,
// exactly as MuNet's CPU and CUDA backends read them (Storage::data(),
// Storage::dtype()); a non-zero status becomes std::runtime_error with the
// library's message.  The backward, loss, optimizer, batch-norm, random and
// all-reduce methods belong to training and are not on the inference path:
// they throw.  query_support reports the library's own table
// (mh_query_support): fp32 / fp16 / bf16 natively, nothing sent to the CPU.
//
// Against a MuNet core carrying munet_core_hip.patch (this directory), whose
// core/backend.hpp declares BackendTransformerCapability, the class also
// provides that capability: LayerNorm, masked_fill, the embedding gather and
// the attention core on the device (mh_layer_norm, mh_masked_fill,
// mh_embedding, mh_attention), which the patched op layer calls instead of
// its host loops.  Against an unpatched core it compiles without it.
//
// Include with MuNet's src/ and this repository's include/ on the path.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "core/backend.hpp"
#include "munet_hip.h"
#include "storage.hpp"

namespace munet {

// The library's dtype and feature codes are MuNet's own enum values.
static_assert(int(DataType::Float32) == MH_F32 && int(DataType::Float16) == MH_F16 &&
                  int(DataType::BFloat16) == MH_BF16 && int(DataType::Int32) == MH_I32,
              "dtype codes");
static_assert(int(BackendFeature::ElementwiseBinary) == MH_FEATURE_ELEMENTWISE_BINARY &&
                  int(BackendFeature::Matmul) == MH_FEATURE_MATMUL &&
                  int(BackendFeature::Convolution) == MH_FEATURE_CONVOLUTION &&
                  int(BackendFeature::Reduction) == MH_FEATURE_REDUCTION,
              "feature codes");
static_assert(int(BackendFallbackPolicy::ExplicitUnsupported) == MH_POLICY_EXPLICIT_UNSUPPORTED &&
                  int(BackendFallbackPolicy::CPUFallback) == MH_POLICY_CPU_FALLBACK,
              "fallback policy codes");

class HIPBackend final : public Backend,
                         public BackendAllocationTransferCapability,
                         public BackendElementwiseCapability,
                         public BackendBlasCapability,
                         public BackendShapeCapability,
#ifdef MUNET_BACKEND_HAS_TRANSFORMER_CAPABILITY
                         public BackendTransformerCapability,
#endif
                         public BackendSpatialCapability {
 public:
  explicit HIPBackend(int index = 0, void *stream = nullptr) : stream_(stream) { check(mh_init(index)); }
  const char *name() const override { return "hip"; }

  BackendAllocationTransferCapability *allocation_transfer_capability() override { return this; }
  const BackendAllocationTransferCapability *allocation_transfer_capability() const override { return this; }
  BackendElementwiseCapability *elementwise_capability() override { return this; }
  const BackendElementwiseCapability *elementwise_capability() const override { return this; }
  BackendBlasCapability *blas_capability() override { return this; }
  const BackendBlasCapability *blas_capability() const override { return this; }
  BackendShapeCapability *shape_capability() override { return this; }
  const BackendShapeCapability *shape_capability() const override { return this; }
  BackendSpatialCapability *spatial_capability() override { return this; }
  const BackendSpatialCapability *spatial_capability() const override { return this; }
#ifdef MUNET_BACKEND_HAS_TRANSFORMER_CAPABILITY
  BackendTransformerCapability *transformer_capability() override { return this; }
  const BackendTransformerCapability *transformer_capability() const override { return this; }
#endif

  BackendSupport query_support(BackendFeature feature, DataType dtype, const Shape *) const override {
    int available = 0, policy = 0, accumulation = 0;
    check(mh_query_support(int(feature), int(dtype), &available, &policy, &accumulation));
    BackendSupport s;
    s.available = available != 0;
    s.fallback_policy = BackendFallbackPolicy(policy);
    s.preferred_accumulation_dtype = DataType(accumulation);
    return s;
  }

  // ---- BackendAllocationTransferCapability (backend.hpp:190-205) ----------
  void *allocate(size_t bytes) override {
    void *p = nullptr;
    check(mh_allocate(&p, bytes));
    return p;
  }
  void deallocate(void *ptr) override { check(mh_deallocate(ptr)); }
  void memset(void *ptr, int value, size_t bytes) override { check(mh_memset(ptr, value, bytes, stream_)); }
  // host endpoints are the CPU device; every other endpoint is this GPU
  void copy(const void *src, void *dst, size_t bytes, Device src_dev, Device dst_dev) override {
    check(mh_copy(src, dst, bytes, endpoint(src_dev), endpoint(dst_dev), stream_));
  }
  void synchronize() override { check(mh_synchronize(stream_)); }
  void all_reduce(Storage &, size_t) override { training_only("all_reduce"); }
  double get_last_kernel_time_us() override { return mh_get_last_kernel_time_us(); }
  bool reports_gpu_kernel_time() const override { return true; }
  void to_contiguous(const Storage &src, Storage &dst, const Shape &shape, const Strides &strides,
                     size_t offset) override {
    const std::vector<int64_t> st(strides.begin(), strides.end());
    check(mh_to_contiguous(code(src), src.data(), dst.data(), int(shape.size()), shape.data(), st.data(),
                           int64_t(offset), stream_));
  }

  // ---- BackendElementwiseCapability (backend.hpp:207-238) ----------------
  void add(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info) override {
    binary(&mh_add, "add", a, b, out, info);
  }
  void sub(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info) override {
    binary(&mh_sub, "sub", a, b, out, info);
  }
  void mul(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info) override {
    binary(&mh_mul, "mul", a, b, out, info);
  }
  void div(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info) override {
    binary(&mh_div, "div", a, b, out, info);
  }
  // dst[r][c] = src[c]: a strided gather with a zero row stride
  void broadcast_row(const Storage &src, Storage &dst, int rows, int cols) override {
    const int shape[2] = {rows, cols};
    const int64_t strides[2] = {0, 1};
    check(mh_to_contiguous(code(src), src.data(), dst.data(), 2, shape, strides, 0, stream_));
  }
  void relu(const Storage &in, Storage &out, size_t n) override { check(mh_relu(code(in), in.data(), out.data(), n, stream_)); }
  void sigmoid(const Storage &in, Storage &out, size_t n) override {
    check(mh_sigmoid(code(in), in.data(), out.data(), n, stream_));
  }
  void exp(const Storage &in, Storage &out, size_t n) override { check(mh_exp(code(in), in.data(), out.data(), n, stream_)); }
  void log(const Storage &in, Storage &out, size_t n) override { check(mh_log(code(in), in.data(), out.data(), n, stream_)); }
  void sqrt(const Storage &in, Storage &out, size_t n) override { check(mh_sqrt(code(in), in.data(), out.data(), n, stream_)); }
  void rsqrt(const Storage &in, Storage &out, size_t n) override {
    check(mh_rsqrt(code(in), in.data(), out.data(), n, stream_));
  }
  void sin(const Storage &in, Storage &out, size_t n) override { check(mh_sin(code(in), in.data(), out.data(), n, stream_)); }
  void cos(const Storage &in, Storage &out, size_t n) override { check(mh_cos(code(in), in.data(), out.data(), n, stream_)); }
  void softmax(const Storage &in, Storage &out, int batch_size, int num_classes) override {
    check(mh_softmax(code(in), in.data(), out.data(), batch_size, num_classes, stream_));
  }
  void relu_backward(const Storage &, const Storage &, Storage &, size_t) override { training_only("relu_backward"); }
  void sigmoid_backward(const Storage &, const Storage &, Storage &, size_t) override {
    training_only("sigmoid_backward");
  }
  void softmax_backward(const Storage &, const Storage &, Storage &, int, int) override {
    training_only("softmax_backward");
  }

  // ---- BackendBlasCapability (backend.hpp:250-260) -----------------------
  void matmul(const Storage &a, const Storage &b, Storage &out, int M, int K, int N, bool transA,
              bool transB) override {
    check(mh_matmul(code(a), a.data(), b.data(), out.data(), M, K, N, transA, transB, stream_));
  }
  void batched_matmul(const Storage &a, const Storage &b, Storage &out, int batch_size, int M, int K, int N,
                      bool transA, bool transB, int64_t stride_a, int64_t stride_b, int64_t stride_out) override {
    check(mh_batched_matmul(code(a), a.data(), b.data(), out.data(), batch_size, M, K, N, transA, transB, stride_a,
                            stride_b, stride_out, stream_));
  }

  // ---- BackendShapeCapability (backend.hpp:263-271) ----------------------
  void concat(const std::vector<Storage *> &inputs, Storage &out, int dim, const std::vector<Shape> &shapes) override {
    if (inputs.empty() || inputs.size() != shapes.size()) throw std::runtime_error("concat: inputs and shapes differ");
    const size_t nd = shapes[0].size();
    std::vector<const void *> ptrs;
    std::vector<int> flat;
    for (size_t i = 0; i < inputs.size(); ++i) {
      if (shapes[i].size() != nd) throw std::runtime_error("concat: inputs of different rank");
      ptrs.push_back(inputs[i]->data());
      flat.insert(flat.end(), shapes[i].begin(), shapes[i].end());
    }
    check(mh_concat(code(out), ptrs.data(), int(inputs.size()), out.data(), dim, int(nd), flat.data(), stream_));
  }
  void concat_backward(const Storage &, std::vector<Storage *> &, int, const std::vector<Shape> &) override {
    training_only("concat_backward");
  }

  // ---- BackendSpatialCapability (backend.hpp:291-311) --------------------
  void conv2d(const Storage &in, const Storage &weight, const Storage *bias, Storage &out, int B, int iC, int iH,
              int iW, int oC, int kH, int kW, int s, int p) override {
    check(mh_conv2d(code(in), in.data(), weight.data(), bias ? bias->data() : nullptr, out.data(), B, iC, iH, iW, oC,
                    kH, kW, s, p, stream_));
  }
  void max_pool2d(const Storage &in, Storage &out, int B, int C, int iH, int iW, int k, int s, int p) override {
    check(mh_max_pool2d(code(in), in.data(), out.data(), B, C, iH, iW, k, s, p, stream_));
  }
  void upsample2d(const Storage &in, Storage &out, int B, int C, int iH, int iW, int scale) override {
    check(mh_upsample2d(code(in), in.data(), out.data(), B, C, iH, iW, scale, stream_));
  }
  void conv2d_backward(const Storage &, const Storage &, const Storage &, Storage &, Storage &, Storage *, int, int,
                       int, int, int, int, int, int, int) override {
    training_only("conv2d_backward");
  }
  void max_pool2d_backward(const Storage &, const Storage &, Storage &, int, int, int, int, int, int, int) override {
    training_only("max_pool2d_backward");
  }
  void upsample2d_backward(const Storage &, Storage &, int, int, int, int, int) override {
    training_only("upsample2d_backward");
  }

#ifdef MUNET_BACKEND_HAS_TRANSFORMER_CAPABILITY
  // ---- BackendTransformerCapability (munet_core_hip.patch) ---------------
  void layer_norm(const Storage &x, const Storage &weight, const Storage &bias, Storage &out, int rows, int cols,
                  float eps) override {
    check(mh_layer_norm(code(x), x.data(), weight.data(), bias.data(), out.data(), rows, cols, eps, stream_));
  }
  void masked_fill(const Storage &x, const Storage &mask, Storage &out, size_t n, double value) override {
    if (mask.dtype() != DataType::Int32) throw std::runtime_error("hip backend: masked_fill takes an Int32 mask");
    check(mh_masked_fill(code(x), x.data(), static_cast<const int32_t *>(mask.data()), out.data(), n, value, stream_));
  }
  // an id outside the table raises the library's device error flag, read
  // back here (a synchronisation) so the call throws the core's message
  void embedding(const Storage &ids, const Storage &weight, Storage &out, int n, int num_embeddings,
                 int dim) override {
    if (ids.dtype() != DataType::Int32) throw std::runtime_error("hip backend: embedding takes Int32 ids");
    check(mh_embedding(code(weight), static_cast<const int32_t *>(ids.data()), weight.data(), out.data(), n,
                       num_embeddings, dim, stream_));
    check(mh_check_device_errors());
  }
  void attention(const Storage &q, const Storage &k, const Storage &v, Storage &merged, int B, int H, int T,
                 int head_dim, bool causal) override {
    check(mh_attention(code(q), q.data(), k.data(), v.data(), merged.data(), B, H, T, head_dim, causal ? 1 : 0,
                       stream_));
  }
#endif

 private:
  void *stream_;

  static void check(int rc) {
    if (rc != 0) throw std::runtime_error(std::string("hip backend: ") + mh_last_error());
  }
  [[noreturn]] static void training_only(const char *op) {
    throw std::runtime_error(std::string("hip backend: ") + op +
                             " is a training operation; the HIP backend runs inference only");
  }
  static int code(const Storage &s) { return static_cast<int>(s.dtype()); }
  static int endpoint(Device d) { return d.type == DeviceType::CPU ? MH_DEVICE_CPU : MH_DEVICE_HIP; }
  using BinaryFn = int (*)(int, const void *, const void *, void *, int, const int *, const int64_t *,
                           const int64_t *, void *);
  void binary(BinaryFn fn, const char *op, const Storage &a, const Storage &b, Storage &out,
              const BroadcastInfo &info) {
    if (!info.can_broadcast) throw std::runtime_error(std::string("hip backend: ") + op + ": shapes do not broadcast");
    const std::vector<int64_t> sa(info.strides_a.begin(), info.strides_a.end());
    const std::vector<int64_t> sb(info.strides_b.begin(), info.strides_b.end());
    check(fn(code(a), a.data(), b.data(), out.data(), int(info.out_shape.size()), info.out_shape.data(), sa.data(),
             sb.data(), stream_));
  }
};

}  // namespace munet
