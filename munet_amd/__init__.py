"""MuNet MI355X HIP backend: hand-written gfx950 kernels behind MuNet's
Backend capability interface and an Engine-style compiled executor.

Submodules:
  _lib      ctypes binding of libmunet_hip.so (include/munet_hip*.h)
  backend   HipBackend, the capability-interface mirror over the C ABI
  engine    Engine (load / compile / run) over the C++ executor
  synth     portable seeded synthetic tensors in MuNet storage formats
  models    module-tree configs and seeded parameters of the workloads
  build     in-tree hipcc build
"""
__all__ = ["_lib", "backend", "engine", "synth", "models", "build"]
