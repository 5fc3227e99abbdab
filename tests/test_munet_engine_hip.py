"""MuNet's own executor on the HIP device.

oracle/_ref/munet_engine_hip (tests/cxx/munet_engine_hip.cpp) is MuNet's core
built from the reference sources with munet_amd/integration/
munet_core_hip.patch applied and MUNET_USE_HIP defined: DeviceType::HIP,
Tensor::to routing, the registry's HIP factory behind the plugin probe, and
the op-layer hooks (BackendTransformerCapability) for LayerNorm, masked_fill,
the embedding gather and attention.  inference::Engine (src/inference.hpp:
292-801) loads, compiles and runs on Device{HIP, 0}:

* the fp32 MLP and CNN (BASELINE configs 1 and 2, full size) from deploy
  artifacts through MuNet's own loader;
* bf16 Linears (2-D and 3-D input: the batched product with stride_b = 0);
* pre-LN TransformerBlocks (bf16 non-causal, fp16 causal) and a two-layer
  bf16 decoder with the embedding gather, built from MuNet's modules.

Each output is compared with the CPU restatement (the oracle) at the
BASELINE tolerances and with the same module's forward on MuNet's CPU
backend in the same process (which equals the oracle bit for bit); two runs
give the same bits.  MUNET_FAIL_FAST_ACCELERATOR_CPU_FALLBACK is set, so any
op that would leave the HIP device for a CPU fallback raises, and the
fallback telemetry must stay at zero.  Tensor::to round trips between host
and device are bit-exact for every dtype.
"""
import os
import subprocess

import numpy as np
import pytest

from munet_amd import models, synth
from oracle import models as omodels
from util import assert_close

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
PATCH = os.path.join(ROOT, "munet_amd", "integration", "munet_core_hip.patch")
BIN = os.path.join(ROOT, "oracle", "_ref", "munet_engine_hip")
# the directory MuNet's plugin loader searches for libmunet_backend_hip.so
PLUGIN_DIR = os.path.join(ROOT, "munet_amd")


def _env():
    env = dict(os.environ)
    env["MUNET_BACKEND_PLUGIN_PATH"] = PLUGIN_DIR
    env["MUNET_FAIL_FAST_ACCELERATOR_CPU_FALLBACK"] = "1"
    return env


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")), reason="reference sources not present")
def test_core_patch_applies_to_the_reference(tmp_path):
    """The patch applies to an unmodified copy of the reference's src/ with
    no fuzz or offset."""
    import shutil
    shutil.copytree(os.path.join(REF, "src"), tmp_path / "src")
    r = subprocess.run(["patch", "-p1", "--dry-run", "-F0", "-i", PATCH], cwd=tmp_path, capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "offset" not in r.stdout and "fuzz" not in r.stdout, r.stdout


@pytest.mark.skipif(not os.path.exists(BIN), reason="oracle/_ref/munet_engine_hip not built (needs the reference)")
def test_no_hip_backend_without_a_gpu(tmp_path):
    """Without a visible GPU the plugin probe fails, MuNet registers no HIP
    backend, and a request for the device fails with the registry's own
    message; the device string still parses."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    (tmp_path / "cases.txt").write_text("")
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, env=_env(), timeout=120)
    assert r.returncode == 1
    lines = r.stdout.splitlines()
    assert lines[0] == "device hip:0 1"
    assert "available hip" not in lines
    # discovered by MuNet's loader, its probe refusing the machine
    assert any(ln.startswith("plugin hip hip runtime_dependency_missing") for ln in lines), lines
    assert lines[-1] == "error Requested backend not compiled or registered."


def _write_params(d, name, p):
    for k, v in p.items():
        np.ascontiguousarray(v).tofile(os.path.join(d, f"{name}.{k}.bin"))


def _cases(d, orc):
    """Writes <d>/cases.txt with its inputs and parameters; returns
    [(name, dtype code, oracle output)]."""
    from munet_amd.artifact import save_deploy_artifact
    cases, lines = [], []

    def add(name, line, cfg, x, ref):
        np.ascontiguousarray(x).tofile(os.path.join(d, f"{name}.x.bin"))
        shape = " ".join(str(v) for v in x.shape)
        lines.append(f"{name} {line} {x.ndim} {shape}")
        cases.append((name, synth.DTYPE_CODES[cfg["dtype"]], ref))

    # BASELINE configs 1 and 2 through MuNet's deploy loader
    for name, cfg, scheme, shape in (("mlp", models.mlp_config(), "mlp", (64, 784)),
                                     ("cnn", models.cnn_config(), "he", (32, 3, 32, 32))):
        p = models.init_params(cfg, scheme, scope=f"me_{name}")
        x = models.make_input(cfg, shape, scheme, scope=f"me_{name}_x")
        path = os.path.join(d, f"{name}.npz")
        save_deploy_artifact(path, cfg, p)
        add(name, f"artifact 0 {path}", cfg, x, omodels.forward(orc, cfg, p, x))
    # bf16 Linears: 2-D, and 3-D input (batched product, stride_b = 0)
    for name, xshape in (("lin2d", (64, 256)), ("lin3d", (4, 48, 256))):
        cfg = models.mlp_config((256, 192), dtype="bfloat16")
        p = models.init_params(cfg, "mlp", scope=f"me_{name}")
        x = models.make_input(cfg, xshape, "mlp", scope=f"me_{name}_x")
        p = {"weight": p["0.weight"], "bias": p["0.bias"]}
        _write_params(d, name, p)
        add(name, "linear 2 256 192", cfg, x, orc.linear(x, p["weight"], p["bias"], synth.BF16))
    # pre-LN blocks and a decoder from MuNet's modules
    for name, cfg, shape in (("block_bf16", models.block_config(128, 4, 512, causal=False, dtype="bfloat16"),
                              (2, 64, 128)),
                             ("block_f16", models.block_config(64, 2, 256, causal=True, dtype="float16"),
                              (3, 48, 64))):
        p = models.init_params(cfg, "xavier", scope=f"me_{name}")
        x = models.make_input(cfg, shape, "xavier", scope=f"me_{name}_x")
        _write_params(d, name, p)
        dtc = synth.DTYPE_CODES[cfg["dtype"]]
        add(name, f"block {dtc} {cfg['d_model']} {cfg['num_heads']} {cfg['ffn']} {int(cfg['causal'])}", cfg, x,
            omodels.forward(orc, cfg, p, x))
    cfg = models.decoder_config(vocab=96, ctx=32, d_model=64, num_heads=4, num_layers=2, ffn=256)
    p = models.init_params(cfg, "gpt", scope="me_dec")
    ids = models.make_input(cfg, (2, 32), "gpt", scope="me_dec_x")
    _write_params(d, "dec", p)
    add("dec", "decoder 2 96 32 64 4 2 256", cfg, ids, omodels.forward(orc, cfg, p, ids))
    with open(os.path.join(d, "cases.txt"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return cases


def _got(d, name, tag, dt, shape):
    return np.fromfile(os.path.join(d, f"{name}.{tag}.bin"), dtype=synth.storage_dtype(dt)).reshape(shape)


@pytest.mark.skipif(not os.path.exists(BIN), reason="oracle/_ref/munet_engine_hip not built (needs the reference)")
def test_cases_on_the_patched_core_cpu(tmp_path, orc):
    """The same cases with the engine on MuNet's CPU device: the patched
    core leaves the CPU path as it was (every output equals the oracle bit
    for bit, the engine's included), and the modules built in the driver
    compose as the oracle does."""
    d = str(tmp_path)
    cases = _cases(d, orc)
    r = subprocess.run([BIN, d, "cpu:0"], capture_output=True, text=True, env=_env(), timeout=600)
    assert r.returncode == 0 and r.stdout.splitlines()[-1] == "ok", r.stdout + r.stderr
    assert "backend cpu" in r.stdout.splitlines()
    for name, dt, ref in cases:
        for tag in ("cpu", "hip", "hip2"):
            assert np.array_equal(_got(d, name, tag, dt, ref.shape), ref), (name, tag)


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(BIN), reason="oracle/_ref/munet_engine_hip not built (needs the reference)")
def test_munet_engine_on_hip_device(tmp_path, orc, hip):
    d = str(tmp_path)
    cases = _cases(d, orc)
    print(f"munet_engine_hip {d}", flush=True)
    r = subprocess.run([BIN, d], capture_output=True, text=True, env=_env(), timeout=300)
    assert r.returncode == 0 and r.stdout.splitlines()[-1] == "ok", r.stdout + r.stderr
    out = r.stdout.splitlines()
    assert out[0] == "device hip:0 1"
    assert "available hip" in out and "backend hip" in out
    assert "plugin hip hip ok" in out
    trips = [ln.split() for ln in out if ln.startswith("roundtrip ")]
    assert len(trips) == 4 and all(t[2:] == ["1", "1", "1"] for t in trips), trips
    assert "accelerator_cpu_fallbacks 0" in out
    for name, dt, ref in cases:
        hip_out, cpu_out = _got(d, name, "hip", dt, ref.shape), _got(d, name, "cpu", dt, ref.shape)
        assert np.array_equal(cpu_out, ref), f"{name}: MuNet's CPU forward differs from the oracle"
        assert_close(hip_out, ref, dt, what=f"MuNet engine on HIP, {name}")
        assert np.array_equal(_got(d, name, "hip2", dt, ref.shape), hip_out), f"{name}: second run differs"
        assert any(ln.startswith(f"case {name} runs 2 ") for ln in out), out
