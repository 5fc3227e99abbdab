// C++ HIP backend with the reference's capability-interface shape.
//
// munet_hip::HipBackend mirrors munet::Backend (reference
// src/core/backend.hpp:347-759) and its capability classes
// (src/core/backend.hpp:190-345): same method names, argument order and
// meaning, operands passed as whole storages (no view offsets or strides
// except BroadcastInfo and to_contiguous), outputs pre-allocated by the
// caller, failures thrown as std::runtime_error.  The storage type here is a
// non-owning view (pointer, bytes, dtype, device) because the reference's
// Storage is not part of this repository; the adapter that binds these
// methods into MuNet's own Backend subclass is shown in INTEGRATION.md.
//
// query_support reports fp32/fp16/bf16 available for every implemented
// feature with fallback ExplicitUnsupported: nothing falls back to the CPU
// (the reference's dtype policy, src/core/backend.hpp:50-71, is fp32-only).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace munet_hip {

enum class DataType { Float32 = 0, Float16 = 1, BFloat16 = 2, Int32 = 3 };
enum class DeviceType { CPU = 0, HIP = 1 };
struct Device {
  DeviceType type = DeviceType::HIP;
  int index = 0;
};

struct Storage {
  void *data = nullptr;
  size_t bytes = 0;
  DataType dtype = DataType::Float32;
  Device device{};
};

using Shape = std::vector<int>;
using Strides = std::vector<int64_t>;

// compute_broadcast result (reference src/types.hpp:419-424).
struct BroadcastInfo {
  Shape out_shape;
  Strides strides_a;
  Strides strides_b;
  bool can_broadcast = false;
};
BroadcastInfo compute_broadcast(const Shape &a_shape, const Strides &a_strides, const Shape &b_shape,
                                const Strides &b_strides);

enum class BackendFeature {
  Elementwise, Matmul, BatchedMatmul, Reduction, Softmax, Concat, Convolution, Pooling, Upsample, ToContiguous,
  LayerNorm, Attention, Embedding, MaskedFill
};
enum class BackendFallbackPolicy { CPUFallback, ExplicitUnsupported };
struct BackendSupport {
  bool available = false;
  BackendFallbackPolicy fallback_policy = BackendFallbackPolicy::ExplicitUnsupported;
  DataType preferred_accumulation_dtype = DataType::Float32;
};

class HipBackend {
 public:
  explicit HipBackend(int device_index = 0, void *stream = nullptr);
  const char *name() const { return "hip"; }
  BackendSupport query_support(BackendFeature feature, DataType dtype, const Shape *shape = nullptr) const;

  // allocation / transfer (backend.hpp:190-205)
  void *allocate(size_t bytes);
  void deallocate(void *ptr);
  void memset(void *ptr, int value, size_t bytes);
  void copy(const void *src, void *dst, size_t bytes, Device src_dev, Device dst_dev);
  void synchronize();
  double get_last_kernel_time_us();
  bool reports_gpu_kernel_time() const { return true; }
  void to_contiguous(const Storage &src, Storage &dst, const Shape &shape, const Strides &strides, size_t offset);

  // elementwise (backend.hpp:207-238)
  void add(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info);
  void sub(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info);
  void mul(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info);
  void div(const Storage &a, const Storage &b, Storage &out, const BroadcastInfo &info);
  void relu(const Storage &in, Storage &out, size_t n);
  void sigmoid(const Storage &in, Storage &out, size_t n);
  void exp(const Storage &in, Storage &out, size_t n);
  void log(const Storage &in, Storage &out, size_t n);
  void sqrt(const Storage &in, Storage &out, size_t n);
  void rsqrt(const Storage &in, Storage &out, size_t n);
  void sin(const Storage &in, Storage &out, size_t n);
  void cos(const Storage &in, Storage &out, size_t n);
  void softmax(const Storage &in, Storage &out, int batch_size, int num_classes);

  // blas (backend.hpp:250-260)
  void matmul(const Storage &a, const Storage &b, Storage &out, int M, int K, int N, bool transA, bool transB);
  void batched_matmul(const Storage &a, const Storage &b, Storage &out, int batch_size, int M, int K, int N,
                      bool transA, bool transB, int64_t stride_a, int64_t stride_b, int64_t stride_out);

  // shape (backend.hpp:263-271)
  void concat(const std::vector<Storage *> &inputs, Storage &out, int dim, const std::vector<Shape> &shapes);

  // spatial (backend.hpp:291-311)
  void conv2d(const Storage &in, const Storage &weight, const Storage *bias, Storage &out, int B, int iC, int iH,
              int iW, int oC, int kH, int kW, int s, int p);
  void max_pool2d(const Storage &in, Storage &out, int B, int C, int iH, int iW, int k, int s, int p);
  void upsample2d(const Storage &in, Storage &out, int B, int C, int iH, int iW, int scale);

  // op-layer functions that have no backend hook in the reference
  void layer_norm(const Storage &x, const Storage &w, const Storage &b, Storage &out, int rows, int cols, float eps);
  void gelu(const Storage &in, Storage &out, size_t n);
  void masked_fill(const Storage &x, const Storage &mask, Storage &out, size_t n, double value);
  void embedding(const Storage &ids, const Storage &weight, Storage &out, int n, int V, int D);
  void attention(const Storage &q, const Storage &k, const Storage &v, Storage &ctx, int B, int H, int T, int hd,
                 bool causal);

 private:
  int device_;
  void *stream_;
};

}  // namespace munet_hip
