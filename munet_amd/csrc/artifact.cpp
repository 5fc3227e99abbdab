// Deploy-artifact loader: MuNet's `munet_model` revision-1 .npz straight into
// an engine (reference load_serialized / parse_and_validate_artifact,
// src/inference_serialization.cpp:902-1080).
//
// The artifact is an uncompressed ZIP of .npy members: one per named
// parameter (Module::named_parameters names) plus `__…__` metadata scalars:
// `__config__` (the module-config JSON the engine takes), `__format_name__`
// "munet_model", `__format_revision__` 1, `__artifact_kind__` "deploy_model",
// `__artifact_scope__` "runtime_only", `__default_load_mode__` "eval",
// `__recommended_loader__` "load_for_inference", `__compile_contract_policy__`
// "external", `__contains_training_state__` False and an optional sorted
// `__tensor_names__` manifest.  The same checks as the reference reject
// anything else, plus tensor names carrying training-state tokens.
//
// One deliberate difference from the reference loader: bf16 tensors (absent
// from the reference, :459-471 and :739-750) are stored as `<u2` arrays of
// bf16 bit patterns; MuNet has no uint16 type, so the mapping is
// unambiguous.  `__producer__`, when present, must be exactly "munet", as the
// reference's C++ loader requires (:997-1000).
//
// The file is memory-mapped; member payloads are handed to
// mh_engine_set_param without an intermediate copy.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "munet_hip.h"
#include "munet_hip_engine.h"
#include "mh_runtime.hpp"

namespace mh {
namespace {

class Mapped {
 public:
  explicit Mapped(const std::string &path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw Error("cannot open artifact '" + path + "'");
    struct stat st;
    if (::fstat(fd_, &st) != 0) throw Error("cannot stat artifact '" + path + "'");
    size_ = size_t(st.st_size);
    if (size_ == 0) throw Error("artifact '" + path + "' is empty");
    void *p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) throw Error("cannot map artifact '" + path + "'");
    data_ = static_cast<const uint8_t *>(p);
  }
  ~Mapped() {
    if (data_) ::munmap(const_cast<uint8_t *>(data_), size_);
    if (fd_ >= 0) ::close(fd_);
  }
  Mapped(const Mapped &) = delete;
  Mapped &operator=(const Mapped &) = delete;
  const uint8_t *data() const { return data_; }
  size_t size() const { return size_; }

 private:
  int fd_ = -1;
  const uint8_t *data_ = nullptr;
  size_t size_ = 0;
};

// Little-endian field readers with bounds checks against the mapped file.
struct Reader {
  const uint8_t *p;
  size_t n;
  void need(uint64_t off, uint64_t len) const {
    if (off > n || len > n - off) throw Error("artifact is truncated or malformed (ZIP structure out of range)");
  }
  uint16_t u16(uint64_t off) const {
    need(off, 2);
    return uint16_t(p[off] | (p[off + 1] << 8));
  }
  uint32_t u32(uint64_t off) const {
    need(off, 4);
    return uint32_t(p[off]) | (uint32_t(p[off + 1]) << 8) | (uint32_t(p[off + 2]) << 16) | (uint32_t(p[off + 3]) << 24);
  }
  uint64_t u64(uint64_t off) const { return uint64_t(u32(off)) | (uint64_t(u32(off + 4)) << 32); }
};

struct Member {
  std::string name;
  const uint8_t *data;
  uint64_t size;
};

// Members of a stored (uncompressed) ZIP archive, ZIP64 sizes included
// (numpy writes every member with ZIP64 local headers).
std::vector<Member> zip_members(const Reader &r) {
  constexpr uint32_t kEocd = 0x06054b50u, kEocd64 = 0x06064b50u, kLoc64 = 0x07064b50u;
  constexpr uint32_t kCentral = 0x02014b50u, kLocal = 0x04034b50u;
  if (r.n < 22) throw Error("artifact is too small to be an .npz archive");
  // end-of-central-directory record: within the last 64 KiB + 22 bytes
  uint64_t eocd = UINT64_MAX;
  const uint64_t lo = r.n > 22 + 65535 ? r.n - 22 - 65535 : 0;
  for (uint64_t pos = r.n - 22 + 1; pos-- > lo;) {
    if (r.u32(pos) == kEocd) {
      eocd = pos;
      break;
    }
  }
  if (eocd == UINT64_MAX) throw Error("artifact has no ZIP central directory (not an .npz archive)");
  uint64_t count = r.u16(eocd + 10), cd_size = r.u32(eocd + 12), cd_off = r.u32(eocd + 16);
  if ((count == 0xffff || cd_size == 0xffffffffu || cd_off == 0xffffffffu) && eocd >= 20 &&
      r.u32(eocd - 20) == kLoc64) {
    const uint64_t z64 = r.u64(eocd - 20 + 8);
    if (r.u32(z64) != kEocd64) throw Error("artifact has a malformed ZIP64 directory record");
    count = r.u64(z64 + 32);
    cd_size = r.u64(z64 + 40);
    cd_off = r.u64(z64 + 48);
  }
  r.need(cd_off, cd_size);
  std::vector<Member> out;
  uint64_t pos = cd_off;
  for (uint64_t i = 0; i < count; ++i) {
    if (r.u32(pos) != kCentral) throw Error("artifact has a malformed ZIP central directory entry");
    const uint16_t method = r.u16(pos + 10);
    uint64_t csize = r.u32(pos + 20), usize = r.u32(pos + 24);
    const uint16_t name_len = r.u16(pos + 28), extra_len = r.u16(pos + 30), comment_len = r.u16(pos + 32);
    uint64_t local = r.u32(pos + 42);
    r.need(pos + 46, uint64_t(name_len) + extra_len + comment_len);
    std::string name(reinterpret_cast<const char *>(r.p + pos + 46), name_len);
    // ZIP64 extended information (header 0x0001): the 8-byte fields present
    // are exactly those whose 32-bit slot holds 0xFFFFFFFF, in this order
    uint64_t e = pos + 46 + name_len;
    const uint64_t e_end = e + extra_len;
    while (e + 4 <= e_end) {
      const uint16_t id = r.u16(e), len = r.u16(e + 2);
      if (id == 0x0001) {
        uint64_t f = e + 4;
        if (usize == 0xffffffffu) { usize = r.u64(f); f += 8; }
        if (csize == 0xffffffffu) { csize = r.u64(f); f += 8; }
        if (local == 0xffffffffu) { local = r.u64(f); f += 8; }
      }
      e += 4 + uint64_t(len);
    }
    if (method != 0) throw Error("artifact member '" + name + "' is compressed; only stored .npz members load");
    if (csize != usize) throw Error("artifact member '" + name + "' has inconsistent sizes");
    if (r.u32(local) != kLocal) throw Error("artifact member '" + name + "' has a malformed local header");
    const uint64_t data = local + 30 + r.u16(local + 26) + r.u16(local + 28);
    r.need(data, usize);
    out.push_back({name, r.p + data, usize});
    pos += 46 + uint64_t(name_len) + extra_len + comment_len;
  }
  return out;
}

// One .npy payload: descr, shape and the raw little-endian data.
struct Npy {
  std::string descr;
  std::vector<uint64_t> shape;
  const uint8_t *data = nullptr;
  uint64_t bytes = 0;
};

std::string header_value(const std::string &h, const std::string &key) {
  const size_t k = h.find("'" + key + "'");
  if (k == std::string::npos) throw Error(".npy header lacks '" + key + "'");
  size_t v = h.find(':', k);
  if (v == std::string::npos) throw Error(".npy header is malformed");
  ++v;
  while (v < h.size() && h[v] == ' ') ++v;
  return h.substr(v);
}

Npy parse_npy(const Member &m) {
  static const uint8_t kMagic[6] = {0x93, 'N', 'U', 'M', 'P', 'Y'};
  if (m.size < 10 || std::memcmp(m.data, kMagic, 6) != 0) throw Error("member '" + m.name + "' is not an .npy array");
  const uint8_t major = m.data[6];
  uint64_t hlen, hoff;
  if (major == 1) {
    hlen = uint64_t(m.data[8]) | (uint64_t(m.data[9]) << 8);
    hoff = 10;
  } else if (major == 2 || major == 3) {
    if (m.size < 12) throw Error("member '" + m.name + "' is truncated");
    hlen = uint64_t(m.data[8]) | (uint64_t(m.data[9]) << 8) | (uint64_t(m.data[10]) << 16) | (uint64_t(m.data[11]) << 24);
    hoff = 12;
  } else {
    throw Error("member '" + m.name + "' uses .npy format version " + std::to_string(major));
  }
  if (hoff + hlen > m.size) throw Error("member '" + m.name + "' has a truncated .npy header");
  const std::string h(reinterpret_cast<const char *>(m.data + hoff), hlen);
  Npy a;
  std::string d = header_value(h, "descr");
  if (d.empty() || d[0] != '\'') throw Error("member '" + m.name + "': descr is not a string");
  a.descr = d.substr(1, d.find('\'', 1) - 1);
  if (header_value(h, "fortran_order").rfind("True", 0) == 0)
    throw Error("member '" + m.name + "' is Fortran-ordered");
  std::string s = header_value(h, "shape");
  if (s.empty() || s[0] != '(') throw Error("member '" + m.name + "': shape is not a tuple");
  s = s.substr(1, s.find(')') - 1);
  size_t i = 0;
  while (i < s.size()) {
    while (i < s.size() && (s[i] == ' ' || s[i] == ',')) ++i;
    if (i >= s.size()) break;
    size_t j = i;
    while (j < s.size() && s[j] >= '0' && s[j] <= '9') ++j;
    if (j == i) throw Error("member '" + m.name + "': bad shape entry");
    a.shape.push_back(std::stoull(s.substr(i, j - i)));
    i = j;
  }
  a.data = m.data + hoff + hlen;
  a.bytes = m.size - hoff - hlen;
  return a;
}

// Element count, or an error when the product of the header's dimensions
// does not fit 64 bits (so it cannot wrap round to match a byte size).
uint64_t elements(const Npy &a) {
  uint64_t n = 1;
  for (uint64_t d : a.shape) {
    if (d != 0 && n > UINT64_MAX / d) throw Error("member shape overflows");
    n *= d;
  }
  return n;
}

bool is_scalar(const Npy &a) { return a.shape.empty() || (a.shape.size() == 1 && a.shape[0] == 1); }

// String metadata: numpy unicode ('<U n', UTF-32LE) or bytes ('|S n').
std::string npy_string(const Npy &a, const std::string &what) {
  if (!is_scalar(a)) throw Error(what + " is not a scalar");
  if (a.descr.size() > 2 && a.descr[1] == 'U') {
    const uint64_t chars = std::stoull(a.descr.substr(2));
    if (chars > a.bytes / 4) throw Error(what + " is truncated");
    std::string out;
    for (uint64_t c = 0; c < chars; ++c) {
      const uint32_t cp = uint32_t(a.data[4 * c]) | (uint32_t(a.data[4 * c + 1]) << 8) |
                          (uint32_t(a.data[4 * c + 2]) << 16) | (uint32_t(a.data[4 * c + 3]) << 24);
      if (cp == 0) break;
      if (cp > 0x7f) throw Error(what + " holds non-ASCII text");
      out.push_back(char(cp));
    }
    return out;
  }
  if (a.descr.size() > 2 && a.descr[1] == 'S') {
    const uint64_t len = std::stoull(a.descr.substr(2));
    if (len > a.bytes) throw Error(what + " is truncated");
    std::string out(reinterpret_cast<const char *>(a.data), len);
    return out.substr(0, out.find('\0'));
  }
  throw Error(what + " is not a string (descr " + a.descr + ")");
}

int64_t npy_int(const Npy &a, const std::string &what) {
  if (!is_scalar(a)) throw Error(what + " is not a scalar");
  if (a.descr == "<i8" && a.bytes >= 8) {
    int64_t v;
    std::memcpy(&v, a.data, 8);
    return v;
  }
  if (a.descr == "<i4" && a.bytes >= 4) {
    int32_t v;
    std::memcpy(&v, a.data, 4);
    return v;
  }
  throw Error(what + " is not an integer (descr " + a.descr + ")");
}

bool npy_bool(const Npy &a, const std::string &what) {
  if (!is_scalar(a) || a.bytes < 1) throw Error(what + " is not a scalar");
  if (a.descr == "|b1" || a.descr == "?" || a.descr == "|?") return a.data[0] != 0;
  throw Error(what + " is not a boolean (descr " + a.descr + ")");
}

// Tensor dtype: the reference's three plus bf16 bit patterns as '<u2'.
int tensor_dtype(const Npy &a, const std::string &name, size_t *elem) {
  if (a.descr == "<f4") { *elem = 4; return MH_F32; }
  if (a.descr == "<f2") { *elem = 2; return MH_F16; }
  if (a.descr == "<u2") { *elem = 2; return MH_BF16; }
  if (a.descr == "<i4") { *elem = 4; return MH_I32; }
  throw Error("tensor '" + name + "' has unsupported dtype " + a.descr);
}

void expect_eq(const std::string &got, const char *want, const char *what) {
  if (got != want) throw Error(std::string("unsupported ") + what + " '" + got + "' (expected '" + want + "')");
}

}  // namespace
}  // namespace mh

extern "C" int mh_engine_create_from_artifact(mh_engine **engine, const char *path, int device) {
  try {
    if (!engine || !path) throw mh::Error("null argument");
    *engine = nullptr;
    mh::Mapped file(path);
    const mh::Reader r{file.data(), file.size()};
    const auto members = mh::zip_members(r);

    std::string format, legacy, producer, kind, scope, mode, loader, policy, config;
    int64_t revision = 0;
    bool training = false, have_manifest = false;
    std::string manifest;
    struct Tensor { std::string name; mh::Npy a; };
    std::vector<Tensor> tensors;
    static const char *kTrainingTokens[] = {"optim", "optimizer", "scheduler", "scaler", "master_weight",
                                           "checkpoint", "epoch", "step", "grad"};
    for (const auto &m : members) {
      std::string name = m.name;
      if (name.size() > 4 && name.compare(name.size() - 4, 4, ".npy") == 0) name.resize(name.size() - 4);
      const mh::Npy a = mh::parse_npy(m);
      if (name.rfind("__", 0) == 0) {
        if (name == "__format_name__") format = mh::npy_string(a, name);
        else if (name == "__format_revision__") revision = mh::npy_int(a, name);
        else if (name == "__format_version__") legacy = mh::npy_string(a, name);
        else if (name == "__producer__") producer = mh::npy_string(a, name);
        else if (name == "__artifact_kind__") kind = mh::npy_string(a, name);
        else if (name == "__artifact_scope__") scope = mh::npy_string(a, name);
        else if (name == "__default_load_mode__") mode = mh::npy_string(a, name);
        else if (name == "__contains_training_state__") training = mh::npy_bool(a, name);
        else if (name == "__recommended_loader__") loader = mh::npy_string(a, name);
        else if (name == "__compile_contract_policy__") policy = mh::npy_string(a, name);
        else if (name == "__config__") config = mh::npy_string(a, name);
        else if (name == "__tensor_names__") { manifest = mh::npy_string(a, name); have_manifest = true; }
        continue;  // other metadata (device / dtype policy) is informational
      }
      std::string low = name;
      std::transform(low.begin(), low.end(), low.begin(), [](unsigned char c) { return char(std::tolower(c)); });
      for (const char *tok : kTrainingTokens)
        if (low.find(tok) != std::string::npos)
          throw mh::Error("deploy artifact carries training state ('" + name + "')");
      tensors.push_back({name, a});
    }
    mh::expect_eq(format, "munet_model", "format name");
    if (revision != 1) throw mh::Error("unsupported format revision " + std::to_string(revision));
    if (!legacy.empty()) mh::expect_eq(legacy, "munet_model_v1", "legacy format tag");
    // exactly the reference's producer tag (src/inference_serialization.cpp:35, :997-1000)
    if (!producer.empty() && producer != "munet") throw mh::Error("unsupported producer '" + producer + "'");
    mh::expect_eq(kind, "deploy_model", "artifact kind");
    mh::expect_eq(scope, "runtime_only", "artifact scope");
    mh::expect_eq(mode, "eval", "default load mode");
    if (training) throw mh::Error("deploy artifact declares training state");
    mh::expect_eq(loader, "load_for_inference", "recommended loader");
    mh::expect_eq(policy, "external", "compile contract policy");
    if (config.empty()) throw mh::Error("deploy artifact has no __config__ (module architecture)");

    std::vector<std::string> names;
    for (const auto &t : tensors) names.push_back(t.name);
    std::sort(names.begin(), names.end());
    if (have_manifest) {
      // the manifest is a JSON array of strings: compare its sorted entries
      std::vector<std::string> listed;
      size_t i = 0;
      while ((i = manifest.find('"', i)) != std::string::npos) {
        const size_t j = manifest.find('"', i + 1);
        if (j == std::string::npos) throw mh::Error("malformed __tensor_names__ manifest");
        listed.push_back(manifest.substr(i + 1, j - i - 1));
        i = j + 1;
      }
      std::sort(listed.begin(), listed.end());
      if (listed != names) throw mh::Error("__tensor_names__ manifest does not match the artifact's tensors");
    }

    mh_engine *e = nullptr;
    if (mh_engine_create(&e, config.c_str(), device) != 0) return 1;
    for (const auto &t : tensors) {
      size_t es = 0;
      const int dt = mh::tensor_dtype(t.a, t.name, &es);
      bool sized = false;
      try {
        sized = t.a.bytes % es == 0 && mh::elements(t.a) == t.a.bytes / es;
      } catch (const std::exception &) {
        sized = false;
      }
      if (!sized) {
        mh_engine_destroy(e);
        throw mh::Error("tensor '" + t.name + "' payload does not match its shape");
      }
      if (mh_engine_set_param(e, t.name.c_str(), t.a.data, t.a.bytes, dt) != 0) {
        const std::string msg = mh_last_error();
        mh_engine_destroy(e);
        throw mh::Error(msg);
      }
    }
    *engine = e;
    return 0;
  } catch (const std::exception &ex) {
    mh::set_last_error(ex.what());
    return 1;
  }
}
