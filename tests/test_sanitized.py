"""The deploy-artifact parser and the compile-time planner under host
AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

tests/cxx/artifact_check.cpp is linked with the library's host sources
(capi.cpp, engine.cpp, artifact.cpp) rebuilt with the sanitizers on their
host code only (hipcc -Xarch_host), and the library's regular kernel objects.
It loads every artifact below on a plan-only engine (parse, validate, lower,
fuse, plan; no GPU) and compiles the valid ones.  The run must be clean (no
sanitizer report), the valid files load and compile, and every malformed one
is refused with a message.
"""
import io
import json
import os
import shutil
import subprocess
import zipfile

import numpy as np
import pytest

from munet_amd import build as hb
from munet_amd import models
from munet_amd.artifact import save_deploy_artifact

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cxx", "_bin")
HOST_SOURCES = ("capi.cpp", "engine.cpp", "artifact.cpp")
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-omit-frame-pointer"]


def _build():
    """The sanitized driver, rebuilt when a source is newer than it."""
    exe = os.path.join(BIN, "artifact_check")
    srcs = [os.path.join(hb.CSRC, s) for s in HOST_SOURCES] + [os.path.join(ROOT, "tests", "cxx", "artifact_check.cpp")]
    srcs += [os.path.join(hb.CSRC, f) for f in os.listdir(hb.CSRC) if f.endswith((".hpp", ".h"))]
    kobjs = [os.path.join(hb.BUILD, s + ".o") for s in hb.KERNEL_SOURCES]
    if not all(os.path.exists(o) for o in kobjs):
        pytest.skip("kernel objects not built (python -m munet_amd.build)")
    if os.path.exists(exe) and os.path.getmtime(exe) > max(os.path.getmtime(p) for p in srcs + kobjs):
        return exe
    os.makedirs(BIN, exist_ok=True)
    hipcc = hb.hipcc()
    flags = ["-O1", "-g", "-std=c++17", "-fPIC", f"--offload-arch={hb.ARCH}", "-I", os.path.join(ROOT, "include"),
             "-I", hb.CSRC] + SAN
    objs = []
    for s in HOST_SOURCES:
        o = os.path.join(BIN, s + ".san.o")
        r = subprocess.run([hipcc] + flags + ["-x", "hip", "-c", os.path.join(hb.CSRC, s), "-o", o],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-3000:]
        objs.append(o)
    r = subprocess.run([hipcc, "-O1", "-g", f"--offload-arch={hb.ARCH}"] + SAN +
                       ["-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "cxx", "artifact_check.cpp"),
                        "-x", "none"] + objs + kobjs + ["-o", exe, "-lpthread"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def _npy(descr, shape, payload):
    hdr = "{'descr': '%s', 'fortran_order': False, 'shape': %s, }" % (descr, shape)
    hdr += " " * ((64 - (10 + len(hdr) + 1) % 64) % 64) + "\n"
    return b"\x93NUMPY\x01\x00" + len(hdr).to_bytes(2, "little") + hdr.encode() + payload


def _zip(path, members):
    with zipfile.ZipFile(path, "w", zipfile.ZIP_STORED) as z:
        for k, v in members.items():
            if isinstance(v, bytes):
                z.writestr(k + ".npy", v)
            else:
                buf = io.BytesIO()
                np.save(buf, v, allow_pickle=False)
                z.writestr(k + ".npy", buf.getvalue())


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_parser_and_planner_under_sanitizers(tmp_path):
    exe = _build()
    files = {}  # name -> (path arg, expect "loaded" / "rejected")

    def good(name, cfg, scheme, shape):
        p = tmp_path / f"{name}.npz"
        save_deploy_artifact(str(p), cfg, models.init_params(cfg, scheme, scope="san"))
        files[name] = (f"{p}:{','.join(map(str, shape))}", "loaded")
        return p

    mlp = good("mlp", models.mlp_config(), "mlp", (4, 784))
    good("cnn", models.cnn_config(), "he", (2, 3, 32, 32))
    good("decoder", models.decoder_config(vocab=300, ctx=32, d_model=64, num_heads=2, num_layers=2, ffn=128),
         "gpt", (2, 32))
    good("unet", models.unet_config(channels=(8, 16, 32), out_channels=2), "he", (1, 3, 32, 32))
    good("encoder", models.block_config(d_model=64, num_heads=4, ffn=128), "xavier", (2, 16, 64))

    raw = mlp.read_bytes()
    with np.load(mlp, allow_pickle=False) as z:
        base = {k: z[k] for k in z.files}

    def bad(name, data):
        p = tmp_path / f"{name}.npz"
        if isinstance(data, dict):
            _zip(p, data)
        else:
            p.write_bytes(data)
        files[name] = (f"{p}:4,784", "rejected")

    bad("empty", b"")
    bad("not_zip", b"\x00" * 200)
    bad("truncated_half", raw[: len(raw) // 2])
    bad("truncated_tail", raw[:-10])
    bad("cd_garbage", raw[:-22] + b"PK\x05\x06" + b"\xff" * 18)
    bad("u_overflow", {**base, "__format_name__": _npy("<U4611686018427387904", "()", b"m\0\0\0")})
    bad("s_overflow", {**base, "__format_name__": _npy("|S18446744073709551615", "()", b"munet_model")})
    bad("shape_overflow", {**base, "0.bias": _npy("<f4", "(4294967296, 4294967296, 1)", b"\0" * 1024)})
    bad("short_payload", {**base, "0.bias": _npy("<f4", "(256,)", b"\0" * 1023)})
    bad("bad_header", {**base, "0.bias": b"\x93NUMPY\x01\x00\xff\xff{'descr'"})
    bad("short_bias", {**base, "0.bias": np.zeros(255, np.float32)})
    bad("short_weight", {**base, "2.weight": np.zeros((256, 255), np.float32)})
    bad("unknown_param", {**base, "9.weight": np.zeros(3, np.float32)})
    bad("int_bias", {**base, "0.bias": np.zeros(256, np.int32)})
    cfg = json.loads(str(base["__config__"]))
    cfg["layers"][0]["in_features"] = -5
    bad("negative_dim", {**base, "__config__": np.array(json.dumps(cfg))})
    bad("config_not_json", {**base, "__config__": np.array("{\"type\": \"Sequential\", \"layers\": [")})

    r = subprocess.run([exe] + [a for a, _ in files.values()], capture_output=True, text=True, timeout=300,
                       env={**os.environ, "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1",
                            "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
    status = {}
    for line in r.stdout.splitlines():
        kind, rest = line.split(" ", 1)
        path = rest.split(":")[0] if kind != "compile" else rest.split(" ", 1)[1].split(":")[0]
        status[os.path.basename(path)[:-4]] = "loaded" if kind == "loaded" else "rejected"
    for name, (_a, want) in files.items():
        assert status.get(name) == want, (name, status.get(name), r.stdout)
