"""Build the MI355X HIP backend libraries in-tree with hipcc (gfx950 only).

Outputs (next to this file):
  libmunet_hip.so             kernels + C ABI + engine (include/munet_hip.h,
                              include/munet_hip_engine.h)
  libmunet_backend_hip.so     MuNet plugin-probe library (5 discovery symbols,
                              reference src/backend/plugin_loader.cpp:122-131)

Run ``python -m munet_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmunet_hip.so")
PLUGIN = os.path.join(HERE, "libmunet_backend_hip.so")
ARCH = "gfx950"

KERNEL_SOURCES = ["gemm.hip", "gemm_pipe.hip", "gemm_pipe_fixed_staged.hip", "gemm_pipe_fixed_dma.hip",
                  "gemm_pipe_wide.hip", "gemm_pipe_conv.hip", "gemm_dma.hip", "attention.hip", "decode.hip",
                  "eltwise.hip", "conv_edge.hip", "gemm_skinny.hip",
                  "norm.hip", "layout.hip", "peak.hip"]
HOST_SOURCES = ["capi.cpp", "engine.cpp", "artifact.cpp"]
PLUGIN_SOURCES = ["plugin.cpp"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm required to build the HIP backend)")


def _flags():
    return [
        "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
        # packed fp32 ops stay off: some of their forms have produced wrong
        # results on these machines
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", os.path.join(ROOT, "include"), "-I", CSRC,
        "-Wno-unused-result",
    ]


# Per-source code-generation options: MFMA results in ordinary VGPRs for the
# attention kernels (the softmax reads every score accumulator with VALU ops;
# accumulation registers would cost a copy per value) and the pipelined GEMM
# (measured faster on MI355X).
_VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
SOURCE_FLAGS = {"attention.hip": _VGPR_FORM, "gemm_pipe.hip": _VGPR_FORM, "gemm_pipe_fixed_staged.hip": _VGPR_FORM,
                "gemm_pipe_fixed_dma.hip": _VGPR_FORM, "gemm_pipe_wide.hip": _VGPR_FORM,
                "gemm_pipe_conv.hip": _VGPR_FORM,
                # the peak loop: with accumulation registers every trip copied
                # each accumulator through ordinary VGPRs
                "peak.hip": _VGPR_FORM}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc()] + _flags() + SOURCE_FLAGS.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [hipcc()] + _flags() + ["-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> None:
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in KERNEL_SOURCES + HOST_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, LIB)
    psrc = [os.path.join(CSRC, s) for s in PLUGIN_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    if psrc:
        tmp = PLUGIN + ".tmp"
        cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-o", tmp] + psrc + ["-ldl"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"plugin build failed: {' '.join(cmd)}\n{res.stderr}")
        os.replace(tmp, PLUGIN)
    if verbose:
        print(f"built {LIB}" + (f" and {PLUGIN}" if psrc else ""))


if __name__ == "__main__":
    build()
    sys.exit(0)
