// Loads each deploy artifact named on the command line with
// mh_engine_create_from_artifact on a plan-only engine (device -1: parse,
// validate, lower, fuse and plan, no GPU) and compiles it for the input
// shape given after it ("path:d0,d1,..."), printing one status line per
// file.  Built with host AddressSanitizer / UndefinedBehaviorSanitizer by
// tests/test_sanitized.py so that the parser and the planner run on
// malformed and valid files under both.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "munet_hip_engine.h"
#include "munet_hip.h"

int main(int argc, char **argv) {
  for (int i = 1; i < argc; ++i) {
    std::string arg = argv[i];
    const size_t colon = arg.rfind(':');
    std::vector<int> shape;
    if (colon != std::string::npos) {
      for (std::string dims = arg.substr(colon + 1); !dims.empty();) {
        const size_t c = dims.find(',');
        shape.push_back(std::atoi(dims.substr(0, c).c_str()));
        dims = c == std::string::npos ? "" : dims.substr(c + 1);
      }
      arg = arg.substr(0, colon);
    }
    mh_engine *e = nullptr;
    if (mh_engine_create_from_artifact(&e, arg.c_str(), -1) != 0) {
      std::printf("rejected %s: %s\n", arg.c_str(), mh_last_error());
      continue;
    }
    if (!shape.empty() && mh_engine_compile(e, shape.data(), int(shape.size())) != 0)
      std::printf("compile failed %s: %s\n", arg.c_str(), mh_last_error());
    else
      std::printf("loaded %s\n", arg.c_str());
    mh_engine_destroy(e);
  }
  return 0;
}
