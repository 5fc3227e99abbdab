// MuNet's own executor on the HIP device: the reference core, built from its
// sources with munet_amd/integration/munet_core_hip.patch applied and
// MUNET_USE_HIP defined (oracle/Makefile, target hipcore), runs
// inference::Engine (src/inference.hpp:292-801) on Device{HIP, 0}.  Nothing
// here calls the HIP library directly: the backend comes from MuNet's own
// registry (register_default_backends, src/backend/backend_manager.cpp:44-79,
// gated by the plugin probe on MUNET_BACKEND_PLUGIN_PATH), parameters move
// through Module::to / Tensor::to, and every op goes through the op layer's
// dispatch (src/core/op_dispatch.cpp:670-718) or the patched op-layer hooks.
//
// usage: munet_engine_hip <dir> [device]
// device defaults to "hip:0"; "cpu:0" runs the same cases with the engine on
// MuNet's CPU backend (a check of the cases and of the patched core's CPU
// behaviour on a machine without a GPU).
// <dir>/cases.txt holds one case per line:
//   <name> artifact <dtype> <path> <ndim> <dims...>   (MuNet's deploy loader)
//   <name> linear   <dtype> <in> <out> <ndim> <dims...>
//   <name> block    <dtype> <d> <heads> <ffn> <causal> <ndim> <dims...>
//   <name> decoder  <dtype> <vocab> <ctx> <d> <heads> <layers> <ffn> <ndim> <dims...>
// dtype is MuNet's DataType value (0 fp32, 1 fp16, 2 bf16).  Inputs are
// <dir>/<name>.x.bin (the input dtype: Int32 ids for the decoder) and, for
// modules built here, <dir>/<name>.<parameter>.bin for every entry of
// named_parameters().  Outputs: <name>.cpu.bin (the same module's forward on
// MuNet's CPU backend, before the engine moves it), <name>.hip.bin and
// <name>.hip2.bin (two Engine::run calls on the HIP device).  The checks of
// the device plumbing (device strings, Tensor::to round trips, the
// registry's backend list, fallback telemetry) are printed on stdout.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "backend/plugin_loader.hpp"
#include "core/backend.hpp"
#include "core/grad_mode.hpp"
#include "core/op_dispatch.hpp"
#include "inference.hpp"
#include "nn/activations.hpp"
#include "nn/attention.hpp"
#include "nn/linear.hpp"
#include "nn/normalization.hpp"
#include "nn/sequential.hpp"
#include "tensor.hpp"

using namespace munet;

namespace {

std::string g_dir;
const Device kCpu{DeviceType::CPU, 0};

std::vector<char> readf(const std::string &name) {
  std::ifstream f(g_dir + "/" + name, std::ios::binary);
  if (!f) throw std::runtime_error("missing input " + name);
  return std::vector<char>(std::istreambuf_iterator<char>(f), {});
}

void writef(const std::string &name, const void *data, size_t bytes) {
  std::ofstream f(g_dir + "/" + name, std::ios::binary);
  f.write(static_cast<const char *>(data), std::streamsize(bytes));
}

void write_tensor(const std::string &name, const Tensor &t) {
  Tensor h = t.to(kCpu).contiguous();
  writef(name, h.data(), h.bytes());
}

Tensor host_tensor(const std::string &file, const Shape &shape, DataType dt) {
  Tensor t(shape, kCpu, dt, false);
  const std::vector<char> bytes = readf(file);
  if (bytes.size() != t.bytes())
    throw std::runtime_error(file + ": " + std::to_string(bytes.size()) + " bytes, expected " +
                             std::to_string(t.bytes()));
  std::memcpy(t.data(), bytes.data(), bytes.size());
  return t;
}

// the pre-LN block of the reference's GPT demo
// (demos/multigpu/gpt3_multi_gpu_demo.py:93-114) from MuNet's modules
class Block : public core::Module {
 public:
  Block(int d, int heads, int ffn, bool causal, TensorOptions o) : core::Module(o) {
    ln1 = register_module("ln1", std::make_shared<nn::LayerNorm>(d, 1e-5f, o));
    attn = register_module("attn", std::make_shared<nn::MultiHeadAttention>(d, heads, causal, o));
    ln2 = register_module("ln2", std::make_shared<nn::LayerNorm>(d, 1e-5f, o));
    auto ff_ = std::make_shared<nn::Sequential>(o);
    ff_->add(std::make_shared<nn::Linear>(d, ffn, true, o));
    ff_->add(std::make_shared<nn::GELU>());
    ff_->add(std::make_shared<nn::Linear>(ffn, d, true, o));
    ff = register_module("ff", ff_);
  }
  Tensor forward_impl(Tensor x) override {
    x = x + attn->forward(ln1->forward(x));
    return x + ff->forward(ln2->forward(x));
  }
  std::shared_ptr<core::Module> ln1, attn, ln2, ff;
};

// the demo's SimpleGPT (:116-172) with Int32 token ids through the
// embedding gather path (src/nn/linear.hpp:95) instead of one-hot inputs
class Decoder : public core::Module {
 public:
  Decoder(int vocab, int ctx, int d, int heads, int layers, int ffn, TensorOptions o) : core::Module(o) {
    // tables without gradients, so nn::Embedding takes its gather path
    auto t = std::make_shared<nn::Embedding>(vocab, d, o), q = std::make_shared<nn::Embedding>(ctx, d, o);
    t->weight.set_requires_grad(false);
    q->weight.set_requires_grad(false);
    tok = register_module("token_embed", t);
    pos = register_module("pos_embed", q);
    for (int i = 0; i < layers; ++i)
      blocks.push_back(register_module("blocks." + std::to_string(i), std::make_shared<Block>(d, heads, ffn, true, o)));
    ln_f = register_module("ln_f", std::make_shared<nn::LayerNorm>(d, 1e-5f, o));
    head = register_module("head", std::make_shared<nn::Linear>(d, vocab, true, o));
  }
  Tensor forward_impl(Tensor ids) override {
    const int B = ids.shape()[0], T = ids.shape()[1];
    Tensor p({B, T}, kCpu, DataType::Int32, false);
    int32_t *pv = static_cast<int32_t *>(p.data());
    for (int b = 0; b < B; ++b)
      for (int t = 0; t < T; ++t) pv[b * T + t] = t;
    Tensor x = tok->forward(ids) + pos->forward(ids.device() == kCpu ? p : p.to(ids.device()));
    for (auto &blk : blocks) x = blk->forward(x);
    return head->forward(ln_f->forward(x));
  }
  std::shared_ptr<core::Module> tok, pos, ln_f, head;
  std::vector<std::shared_ptr<core::Module>> blocks;
};

// Module::parse_device_string is protected: the device-string parser that
// Module::offload uses (src/core/module.hpp:653-683)
struct DeviceSpec : core::Module {
  static Device parse(const std::string &s) { return parse_device_string(s); }
  Tensor forward_impl(Tensor x) override { return x; }
};

void load_params(const std::string &name, core::Module &m) {
  for (auto &[pname, p] : m.named_parameters()) {
    Tensor src = host_tensor(name + "." + pname + ".bin", p.shape(), p.dtype());
    std::memcpy(p.data(), src.data(), p.bytes());
  }
}

Shape read_shape(std::istringstream &in) {
  int nd = 0;
  in >> nd;
  Shape s(nd);
  for (int &v : s) in >> v;
  if (!in) throw std::runtime_error("bad shape in cases.txt");
  return s;
}

void run_case(const std::string &line, const Device &dev) {
  std::istringstream in(line);
  std::string name, kind;
  int dtc = 0;
  in >> name >> kind >> dtc;
  const DataType dt = DataType(dtc);
  TensorOptions o = TensorOptions{}.with_device(kCpu).with_dtype(dt);
  std::shared_ptr<core::Module> m;
  DataType in_dt = dt;
  if (kind == "artifact") {
    std::string path;
    in >> path;
    m = inference::load_serialized(path, kCpu);
  } else if (kind == "linear") {
    int fin = 0, fout = 0;
    in >> fin >> fout;
    m = std::make_shared<nn::Linear>(fin, fout, true, o);
  } else if (kind == "block") {
    int d = 0, h = 0, f = 0, causal = 0;
    in >> d >> h >> f >> causal;
    m = std::make_shared<Block>(d, h, f, causal != 0, o);
  } else if (kind == "decoder") {
    int v = 0, c = 0, d = 0, h = 0, l = 0, f = 0;
    in >> v >> c >> d >> h >> l >> f;
    m = std::make_shared<Decoder>(v, c, d, h, l, f, o);
    in_dt = DataType::Int32;
  } else {
    throw std::runtime_error("unknown case kind " + kind);
  }
  const Shape xs = read_shape(in);
  if (kind != "artifact") load_params(name, *m);
  m->eval();
  const Tensor x = host_tensor(name + ".x.bin", xs, in_dt);

  // MuNet's CPU backend first (the engine moves the module's parameters)
  {
    NoGradGuard ng;
    write_tensor(name + ".cpu.bin", m->forward(x));
  }

  inference::EngineConfig cfg;
  cfg.device = dev;
  inference::Engine eng(cfg);
  eng.load(m);
  if (!m->is_on(dev)) throw std::runtime_error(name + ": parameters not on " + dev.to_string());
  eng.compile(x);
  const Tensor y = eng.run(x);
  if (y.device() != dev) throw std::runtime_error(name + ": output on " + y.device().to_string());
  write_tensor(name + ".hip.bin", y);
  write_tensor(name + ".hip2.bin", eng.run(x));
  const inference::EngineStats st = eng.stats();
  std::printf("case %s runs %zu cache_hits %zu out_shape", name.c_str(), st.runs, st.prepared_input_cache_hits);
  for (int v : y.shape()) std::printf(" %d", v);
  std::printf("\n");
  std::fflush(stdout);
}

// Tensor::to between the host and the device and back, bit for bit, for
// every dtype, from a contiguous and from a transposed (strided) source
void round_trips(const Device &hip) {
  for (DataType dt : {DataType::Float32, DataType::Float16, DataType::BFloat16, DataType::Int32}) {
    Tensor h({37, 29}, kCpu, dt, false);
    unsigned char *b = static_cast<unsigned char *>(h.data());
    for (size_t i = 0; i < h.bytes(); ++i) b[i] = static_cast<unsigned char>((i * 131 + 7) ^ (i >> 5));
    Tensor d = h.to(hip);
    if (d.device() != hip) throw std::runtime_error("Tensor::to(hip) left the tensor on " + d.device().to_string());
    Tensor back = d.to(kCpu);
    const bool same = std::memcmp(back.data(), h.data(), h.bytes()) == 0;
    Tensor tv = h.transpose(0, 1).to(hip).to(kCpu);  // packed on the host, then moved
    Tensor tr = h.transpose(0, 1).contiguous();
    const bool same_t = std::memcmp(tv.data(), tr.data(), tr.bytes()) == 0;
    Tensor dd = d.to(Device{DeviceType::HIP, 0}).to(kCpu);  // same device: no copy
    const bool same_d = std::memcmp(dd.data(), h.data(), h.bytes()) == 0;
    std::printf("roundtrip %d %d %d %d\n", int(dt), int(same), int(same_t), int(same_d));
  }
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 2 && argc != 3) {
    std::fprintf(stderr, "usage: munet_engine_hip <dir> [device]\n");
    return 2;
  }
  g_dir = argv[1];
  try {
    const Device hip = DeviceSpec::parse("hip:0");
    std::printf("device %s %d\n", hip.to_string().c_str(), int(hip.type == DeviceType::HIP));
    for (const auto &st : plugin::plugins_for_device("hip"))
      std::printf("plugin %s %s %s\n", st.name.c_str(), st.device.c_str(), st.reason_code.c_str());
    for (const std::string &b : BackendManager::list_available_backends()) std::printf("available %s\n", b.c_str());
    const Device dev = DeviceSpec::parse(argc == 3 ? argv[2] : "hip:0");
    std::printf("backend %s\n", BackendManager::get(dev)->name());
    std::fflush(stdout);
    if (dev.type == DeviceType::HIP) round_trips(dev);
    const std::vector<char> text = readf("cases.txt");
    std::istringstream cases(std::string(text.begin(), text.end()));
    for (std::string line; std::getline(cases, line);)
      if (!line.empty()) run_case(line, dev);
    const ops::FallbackTelemetrySnapshot t = ops::fallback_telemetry_snapshot();
    std::printf("accelerator_cpu_fallbacks %llu\n", static_cast<unsigned long long>(t.accelerator_cpu_fallback_total));
    for (const auto &[k, v] : t.accelerator_cpu_fallback_counters)
      std::printf("fallback %s %llu\n", k.c_str(), static_cast<unsigned long long>(v));
    std::printf("ok\n");
  } catch (const std::exception &e) {
    std::printf("error %s\n", e.what());
    return 1;
  }
  return 0;
}
