// MuNet backend-plugin discovery library for the HIP backend
// (libmunet_backend_hip.so).  MuNet's plugin loader dlopens
// libmunet_backend_<name>.so, reads these five symbols, probes, and dlcloses
// (reference src/backend/plugin_loader.cpp:101-176, ABI version 1 at
// src/backend/plugin_loader.hpp:9).  Compute stays in libmunet_hip.so.
//
// The probe loads the HIP runtime and asks for a device: nullptr means the
// backend is usable, otherwise a reason string.
#include <dlfcn.h>

#include <cstdint>

extern "C" {

uint32_t munet_backend_plugin_abi_version(void) { return 1u; }
const char *munet_backend_plugin_name(void) { return "hip"; }
const char *munet_backend_plugin_device_type(void) { return "hip"; }

const char *munet_backend_plugin_probe(void) {
  void *rt = dlopen("libamdhip64.so", RTLD_NOW | RTLD_LOCAL);
  if (!rt) rt = dlopen("/opt/rocm/lib/libamdhip64.so", RTLD_NOW | RTLD_LOCAL);
  if (!rt) return "runtime_dependency_missing: libamdhip64.so";
  typedef int (*count_fn)(int *);
  count_fn f = reinterpret_cast<count_fn>(dlsym(rt, "hipGetDeviceCount"));
  int n = 0;
  const bool ok = f && f(&n) == 0 && n > 0;
  dlclose(rt);
  return ok ? nullptr : "no HIP device visible";
}

// bit 0 elementwise, 1 blas, 2 spatial, 3 shape, 4 layer norm, 5 attention,
// 6 embedding; bits 16-18 fp32 / fp16 / bf16 storage.
uint64_t munet_backend_plugin_capability_flags(void) { return 0x7fULL | (0x7ULL << 16); }

}  // extern "C"
