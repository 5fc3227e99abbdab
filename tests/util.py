"""Parity helpers shared by the tests (tolerances from BASELINE.json north_star)."""
import numpy as np

from munet_amd import synth

RTOL = {synth.F32: 1e-4, synth.F16: 2e-2, synth.BF16: 2e-2}


def dec(x, dt):
    return synth.decode(x, dt).astype(np.float64)


def normwise_err(y, y_ref, dt):
    a, b = dec(y, dt), dec(y_ref, dt)
    assert a.shape == b.shape, (a.shape, b.shape)
    scale = np.max(np.abs(b)) if b.size else 0.0
    if scale == 0:
        scale = 1.0
    return float(np.max(np.abs(a - b)) / scale) if a.size else 0.0


def assert_close(y, y_ref, dt, rtol=None, what=""):
    """max|y - y_ref| <= rtol * max|y_ref| (normwise), rtol 1e-4 fp32, 2e-2 fp16/bf16."""
    rtol = RTOL[dt] if rtol is None else rtol
    assert np.all(np.isfinite(dec(y, dt)) == np.isfinite(dec(y_ref, dt))), f"{what}: non-finite mismatch"
    err = normwise_err(y, y_ref, dt)
    assert err <= rtol, f"{what}: normwise error {err:.3e} > {rtol:.1e}"
    return err


def rand(shape, dt, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return synth.encode(rng.standard_normal(shape) * scale, dt)
