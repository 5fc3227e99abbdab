// Host runtime helpers shared by the C ABI and the engine: error type, HIP
// status checks, per-device error flag and growable workspace.
#pragma once

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

namespace mh {

struct Error : std::runtime_error {
  explicit Error(const std::string &m) : std::runtime_error(m) {}
};

void set_last_error(const std::string &msg);
void hip_check(hipError_t e, const char *what);
int current_device();
int *device_error_flag();
// Grow-only scratch on the current device (may hipMalloc; never under capture).
void *workspace(size_t bytes);
void set_last_kernel_time_us(double us);

}  // namespace mh
