"""Static check of the direct-to-LDS GEMM's first wait (CPU; needs hipcc).

The kernel issues the loads of slabs 0 .. S-2 with inline assembly
(global_load_lds_dwordx4; a convolution's A blocks through
buffer_load_dwordx4 ... lds), after the optional 4-byte loads that touch the
next GEMM's weights, then, for the fixed epilogue programs, the bias /
residual prefetch, and waits with ``s_waitcnt vmcnt(N)`` for slab 0.  vmcnt
counts outstanding vector-memory operations and they complete in order, so
slab 0 has landed exactly when N is at most the number of vector-memory
operations issued after slab 0's last load.  N is a compile-time count in
the source (NDMA * (S - 2) + the prefetch's load count); this test compiles
the kernels to gfx950 assembly and checks it against the instructions the
compiler actually emitted, for every instantiation."""
import os
import re
import shutil
import subprocess

import pytest

from munet_amd import build

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _asm(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = [HIPCC] + build._flags() + build.SOURCE_FLAGS.get(src, []) + [
        "--cuda-device-only", "-S", os.path.join(build.CSRC, src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _template_args(name):
    # integer arguments, then the convolution flag (Lb0E / Lb1E)
    m = re.search(r"gemm_dma_kernelI((?:Li-?\d+E)+)(?:Lb[01]E)?E", name)
    return [int(v) for v in re.findall(r"Li(-?\d+)E", m.group(1))]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src", ["gemm_pipe_wide.hip", "gemm_pipe_fixed_dma.hip", "gemm_pipe_conv.hip"])
def test_first_slab_wait_covers_slab0(src, tmp_path):
    s = _asm(src, tmp_path)
    checked = 0
    for m in re.finditer(r"^(_Z\S*gemm_dma_kernel\S*):", s, re.M):
        name = m.group(1)
        dt, bm, bn, wgm, wgn, stages, ek = _template_args(name)
        body = s[m.end():s.index(".Lfunc_end", m.end())]
        ins = [ln.strip() for ln in body.splitlines()
               if ln.strip() and not ln.strip().startswith((";", ".")) and not re.match(r"^\S+:$", ln.strip())]
        first_mfma = next(i for i, x in enumerate(ins) if "mfma" in x)
        pro = ins[:first_mfma]
        # the slabs' 16-byte DMAs (the 4-byte loads issued before them touch
        # the next GEMM's weights; being older, they only add to the wait)
        # (convolutions: the A blocks through the buffer form, padding taps
        # landing as zeros)
        dma = [i for i, x in enumerate(pro)
               if x.startswith("global_load_lds_dwordx4") or (x.startswith("buffer_load_dwordx4") and x.endswith(" lds"))]
        assert dma and len(dma) % (stages - 1) == 0, (name, len(dma))
        ndma = len(dma) // (stages - 1)
        last0 = dma[ndma - 1]  # slab 0's last load
        wait = next(i for i, x in enumerate(pro) if i > dma[-1] and re.match(r"s_waitcnt\b.*vmcnt\(\d+\)", x))
        n = int(re.search(r"vmcnt\((\d+)\)", pro[wait]).group(1))
        later = [x for x in pro[last0 + 1:wait]
                 if re.match(r"(global|buffer|flat)_load", x)]
        assert n <= len(later), f"{name}: vmcnt({n}) with {len(later)} loads after slab 0"
        checked += 1
    assert checked > 0
