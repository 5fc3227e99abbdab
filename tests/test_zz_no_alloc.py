"""mh_matmul_noalloc, the matmul entry point for callers that cannot allocate:
it must compute exactly what mh_matmul computes (the same transposes and
GEMM kernels, staged in the library's fixed per-device scratch instead of the
growable workspace), on consecutive calls of shrinking size (the scratch
keeps the previous call's contents), never take device memory, and refuse
a call whose staging exceeds the scratch before enqueuing anything."""
import numpy as np
import pytest

from munet_amd import synth
from munet_amd._lib import HipError
from munet_amd.backend import empty, to_device, to_host
from util import assert_close, rand

pytestmark = pytest.mark.gpu

DTS = [synth.F32, synth.F16, synth.BF16]


def _operands(M, K, N, ta, tb, dt, seed):
    a = rand((M, K), dt, seed)
    b = rand((K, N), dt, seed + 1)
    a_st = synth.encode(np.ascontiguousarray(synth.decode(a, dt).T), dt) if ta else a
    b_st = synth.encode(np.ascontiguousarray(synth.decode(b, dt).T), dt) if tb else b
    return a, b, to_device(a_st, dt), to_device(b_st, dt)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (1, 1), (0, 1)])
def test_noalloc_matches_matmul_on_shrinking_calls(hip, orc, dt, ta, tb):
    import torch
    for i, (M, K, N) in enumerate(((300, 520, 260), (37, 65, 19))):
        print(f"noalloc dt={dt} t{ta}{tb} call {i}: {M}x{K}x{N}", flush=True)
        a, b, ad, bd = _operands(M, K, N, ta, tb, dt, 40 + i)
        got = empty((M, N), dt)
        hip.matmul_noalloc(ad, bd, got, M, K, N, bool(ta), bool(tb))
        want = empty((M, N), dt)
        hip.matmul(ad, bd, want, M, K, N, bool(ta), bool(tb))
        torch.cuda.synchronize()
        assert np.array_equal(to_host(got, dt), to_host(want, dt)), f"call {i} differs from mh_matmul"
        assert_close(to_host(got, dt), orc.matmul(a, b, dt), dt, what=f"noalloc call {i}")


def test_noalloc_takes_no_device_memory(hip):
    """A call staging ~48 MiB of transposed operands leaves the device's free
    memory where it was (mh_matmul would grow its workspace by that much)."""
    import torch
    dt = synth.BF16
    M, K, N = 64, 4096, 6144  # B [K,N] transposed: 48 MiB of staging
    small = _operands(8, 16, 8, 0, 0, dt, 60)
    out = empty((8, 8), dt)
    hip.matmul_noalloc(small[2], small[3], out, 8, 16, 8, False, False)
    a = to_device(rand((M, K), dt, 61), dt)
    b = to_device(rand((K, N), dt, 62, 0.02), dt)
    big = empty((M, N), dt)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    hip.matmul_noalloc(a, b, big, M, K, N, False, False)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free0 - free1 < (8 << 20), f"device free memory fell by {(free0 - free1) >> 20} MiB"


def test_noalloc_rejects_staging_beyond_scratch(hip):
    """B [6000, 6000] bf16 transposed needs 72 MB > the 64 MiB scratch: an
    error before any launch (the tiny buffers are never touched)."""
    dt = synth.BF16
    tiny = to_device(np.zeros(16, np.uint16), dt)
    with pytest.raises(HipError, match="more than its fixed"):
        hip.matmul_noalloc(tiny, tiny, tiny, 8, 6000, 6000, False, False)
    with pytest.raises(HipError, match="more than its fixed"):
        hip.matmul_noalloc(tiny, tiny, tiny, 6000, 6000, 8, True, True)
