// Drives munet::HIPBackend (munet_amd/integration/munet_hip_backend.hpp)
// through MuNet's own compiled registry and storages: the adapter is
// registered with BackendManager for the CUDA device slot (the way the
// reference's tests swap a device's backend, tests/test_backend_manager.cpp:
// 122-130; DeviceType has no HIP value until a MuNet build adds one),
// munet::Storage objects allocate through it, host data moves through its
// copy(), and the ops run through Backend's forwarding methods
// (src/core/backend.hpp:447-715).  Inputs are raw files written by
// tests/test_adapter.py in <dir>; outputs are written back there, and the
// support table and error behaviour are printed on stdout.
#include <cstdio>
#include <fstream>
#include <iterator>
#include <memory>
#include <string>
#include <vector>

#include "munet_hip_backend.hpp"
#include "types.hpp"

using namespace munet;

namespace {

std::string g_dir;

std::vector<char> readf(const std::string &name) {
  std::ifstream f(g_dir + "/" + name, std::ios::binary);
  if (!f) throw std::runtime_error("missing input " + name);
  return std::vector<char>(std::istreambuf_iterator<char>(f), {});
}

void writef(const std::string &name, const std::vector<char> &bytes) {
  std::ofstream f(g_dir + "/" + name, std::ios::binary);
  f.write(bytes.data(), std::streamsize(bytes.size()));
}

Strides contiguous(const Shape &s) {
  Strides st(s.size(), 1);
  for (int i = int(s.size()) - 2; i >= 0; --i) st[i] = st[i + 1] * s[i + 1];
  return st;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: adapter_check <dir>\n");
    return 2;
  }
  g_dir = argv[1];
  try {
    BackendManager::registry().clear_cache(DeviceType::CUDA);
    BackendManager::register_backend(DeviceType::CUDA,
                                     [](Device d) { return std::make_shared<HIPBackend>(d.index); });
    const Device gpu{DeviceType::CUDA, 0}, cpu{DeviceType::CPU, 0};
    std::shared_ptr<Backend> be = BackendManager::get(gpu);
    std::printf("backend %s\n", be->name());

    auto up = [&](const std::string &name, DataType dt, const Shape &shape) {
      const std::vector<char> h = readf(name);
      auto s = std::make_unique<Storage>(h.size(), gpu, dt, shape);
      be->copy(h.data(), s->data(), h.size(), cpu, gpu);
      return s;
    };
    auto out = [&](size_t bytes, DataType dt, const Shape &shape) {
      return std::make_unique<Storage>(bytes, gpu, dt, shape);
    };
    auto down = [&](const std::string &name, const Storage &s) {
      std::vector<char> h(s.size_bytes());
      be->copy(s.data(), h.data(), h.size(), gpu, cpu);
      be->synchronize();
      writef(name, h);
    };

    // matmul bf16 [64,96] x [96,80], and with B stored transposed [80,96]
    auto a = up("mm_a.bin", DataType::BFloat16, {64, 96});
    auto b = up("mm_b.bin", DataType::BFloat16, {96, 80});
    auto bt = up("mm_bt.bin", DataType::BFloat16, {80, 96});
    auto c = out(64 * 80 * 2, DataType::BFloat16, {64, 80});
    be->matmul(*a, *b, *c, 64, 96, 80, false, false);
    down("out_mm.bin", *c);
    be->matmul(*a, *bt, *c, 64, 96, 80, false, true);
    down("out_mm_t.bin", *c);

    // add fp16 with broadcast [4,5,6] + [6], strides from MuNet's compute_broadcast
    auto x = up("add_a.bin", DataType::Float16, {4, 5, 6});
    auto y = up("add_b.bin", DataType::Float16, {6});
    const BroadcastInfo bi = compute_broadcast({4, 5, 6}, contiguous({4, 5, 6}), {6}, contiguous({6}));
    auto z = out(4 * 5 * 6 * 2, DataType::Float16, {4, 5, 6});
    be->add(*x, *y, *z, bi);
    down("out_add.bin", *z);

    // conv2d fp32 [2,3,9,9] * [4,3,3,3] + bias, stride 1, pad 1
    auto ci = up("conv_x.bin", DataType::Float32, {2, 3, 9, 9});
    auto cw = up("conv_w.bin", DataType::Float32, {4, 3, 3, 3});
    auto cb = up("conv_b.bin", DataType::Float32, {4});
    auto co = out(2 * 4 * 9 * 9 * 4, DataType::Float32, {2, 4, 9, 9});
    be->conv2d(*ci, *cw, cb.get(), *co, 2, 3, 9, 9, 4, 3, 3, 1, 1);
    down("out_conv.bin", *co);

    // softmax fp32 [7, 33]
    auto si = up("sm_x.bin", DataType::Float32, {7, 33});
    auto so = out(7 * 33 * 4, DataType::Float32, {7, 33});
    be->softmax(*si, *so, 7, 33);
    down("out_sm.bin", *so);

    // max_pool2d fp16 [2,3,8,8], k 2 s 2
    auto pi = up("pool_x.bin", DataType::Float16, {2, 3, 8, 8});
    auto po = out(2 * 3 * 4 * 4 * 2, DataType::Float16, {2, 3, 4, 4});
    be->max_pool2d(*pi, *po, 2, 3, 8, 8, 2, 2, 0);
    down("out_pool.bin", *po);

    // broadcast_row int32 [5] -> [3, 5]
    auto ri = up("row_x.bin", DataType::Int32, {5});
    auto ro = out(3 * 5 * 4, DataType::Int32, {3, 5});
    be->broadcast_row(*ri, *ro, 3, 5);
    down("out_row.bin", *ro);

    // concat bf16 along dim 1: [2,3,4] ++ [2,5,4]
    auto k0 = up("cat_a.bin", DataType::BFloat16, {2, 3, 4});
    auto k1 = up("cat_b.bin", DataType::BFloat16, {2, 5, 4});
    auto ko = out(2 * 8 * 4 * 2, DataType::BFloat16, {2, 8, 4});
    be->concat({k0.get(), k1.get()}, *ko, 1, {{2, 3, 4}, {2, 5, 4}});
    down("out_cat.bin", *ko);

    // the support table MuNet's dispatch would see
    for (int f = 0; f <= int(BackendFeature::Reduction); ++f)
      for (int d = 0; d <= int(DataType::Int32); ++d) {
        const BackendSupport s = be->query_support(BackendFeature(f), DataType(d));
        std::printf("support %d %d %d %d %d\n", f, d, int(s.available), int(s.fallback_policy),
                    int(s.preferred_accumulation_dtype));
      }
    // a training method throws, the storage stays usable
    try {
      be->relu_backward(*si, *si, *so, 7 * 33);
      std::printf("relu_backward did not throw\n");
    } catch (const std::exception &e) {
      std::printf("training_only %s\n", e.what());
    }
    std::printf("ok\n");
  } catch (const std::exception &e) {
    std::printf("error %s\n", e.what());
    return 1;
  }
  return 0;
}
