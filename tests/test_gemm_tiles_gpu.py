"""Every GEMM block-tile variant (direct-to-LDS, general register-staged and
pipelined) against the oracle, forced through MUNET_HIP_GEMM_TILE in a child
process, on shapes with ragged M / N tails, N % 4 != 0 (general epilogue),
K from one to seven 64-wide slabs and ragged K (short first slab)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))

SCRIPT = r'''
import sys, numpy as np
sys.path.insert(0, {root!r}); sys.path.insert(0, {tests!r})
import torch
from munet_amd.backend import HipBackend, empty, to_device, to_host
from munet_amd import synth
from oracle import CpuOracle
from util import assert_close, rand
hip, orc = HipBackend(0), CpuOracle("restatement")
for dt in (synth.BF16, synth.F16):
    for (M, K, N) in [(300, 192, 200), (257, 128, 129), (64, 64, 64), (520, 256, 264), (96, 200, 72),
                      (130, 320, 96), (70, 448, 136), (33, 40, 48)]:
        x, w, b = rand((M, K), dt, 1), rand((K, N), dt, 2, 0.2), rand((N,), dt, 3)
        r = rand((M, N), dt, 4)
        ref = orc.add(r, orc.gelu(orc.linear(x, w, b, dt), dt), dt)
        wt = empty((N, K), dt)
        hip.pack_linear_weight(to_device(w, dt), wt, K, N)
        out = empty((M, N), dt)
        hip.linear(to_device(x, dt), wt, to_device(b, dt), out, M, K, N, 2, to_device(r, dt))
        assert_close(to_host(out, dt), ref, dt, what=f"tile={tile} dt={{dt}} {{M}}x{{K}}x{{N}}")
print("ok")
'''


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 5, 6, 100, 101, 102, 103, 104, 105, 106, 107, 200, 201, 202, 203])
def test_forced_tile(tile):
    root = os.path.dirname(HERE)
    code = SCRIPT.format(root=root, tests=HERE, tile=tile)
    env = dict(os.environ, MUNET_HIP_GEMM_TILE=str(tile))
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and "ok" in res.stdout, res.stdout[-2000:] + res.stderr[-2000:]
