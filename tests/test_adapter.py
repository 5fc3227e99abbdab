"""The MuNet Backend adapter (munet_amd/integration/munet_hip_backend.hpp):

* CPU: it compiles against MuNet's own headers and is a concrete class (every
  pure virtual of the capabilities it provides is implemented), when the
  reference sources are present;
* GPU: oracle/_ref/adapter_check (tests/cxx/adapter_check.cpp, linked against
  MuNet's compiled CPU sources and libmunet_hip.so) registers it with MuNet's
  BackendManager, allocates munet::Storage objects through it and runs
  matmul, broadcast add, conv2d, softmax, max_pool2d, broadcast_row and concat
  through Backend's forwarding methods; the outputs are compared with the
  oracle, and the support table it reports with mh_query_support.
"""
import os
import subprocess

import numpy as np
import pytest

from munet_amd import synth
from munet_amd.backend import FEATURES, query_support
from oracle import CpuOracle
from util import assert_close, rand

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
ADAPTER = os.path.join(ROOT, "munet_amd", "integration", "munet_hip_backend.hpp")
CHECK = os.path.join(ROOT, "oracle", "_ref", "adapter_check")


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")), reason="reference sources not present")
def test_adapter_compiles_against_munet_headers(tmp_path):
    tu = tmp_path / "tu.cpp"
    tu.write_text('#include "munet_hip_backend.hpp"\n#include <type_traits>\n'
                  'static_assert(!std::is_abstract<munet::HIPBackend>::value, "pure virtual left");\n'
                  'static_assert(std::is_base_of<munet::Backend, munet::HIPBackend>::value, "not a Backend");\n')
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror", f"-I{REF}/src",
                        f"-I{ROOT}/include", f"-I{os.path.dirname(ADAPTER)}", str(tu)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_query_support_table():
    """fp32/fp16/bf16 for the float kernels, int32 too for data movement,
    training and reduction features unavailable, ExplicitUnsupported and fp32
    accumulation everywhere (the reference's contract,
    src/core/backend.hpp:411-425)."""
    floats = {"elementwise_binary", "matmul", "unary_activation", "softmax", "convolution", "pooling",
              "layer_norm", "attention", "embedding", "masked_fill"}
    movement = {"broadcast_row", "concat", "to_contiguous"}
    for f in FEATURES:
        for dt in (synth.F32, synth.F16, synth.BF16, synth.I32):
            s = query_support(f, dt)
            want = (f in floats and dt != synth.I32) or f in movement
            assert s.available == want, (f, dt)
            assert s.fallback_policy == "ExplicitUnsupported" and s.preferred_accumulation_dtype == synth.F32
    assert not query_support("no_such_feature", synth.F32).available
    from munet_amd._lib import HipError
    with pytest.raises(HipError, match="unsupported dtype"):
        query_support("matmul", 9)


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(CHECK), reason="oracle/_ref/adapter_check not built (needs the reference)")
def test_adapter_through_munet_storages(tmp_path, orc, hip):
    F32, F16, BF16, I32 = synth.F32, synth.F16, synth.BF16, synth.I32
    d = str(tmp_path)
    ins = {
        "mm_a": rand((64, 96), BF16, 300), "mm_b": rand((96, 80), BF16, 301, 0.2),
        "add_a": rand((4, 5, 6), F16, 302), "add_b": rand((6,), F16, 303),
        "conv_x": rand((2, 3, 9, 9), F32, 304), "conv_w": rand((4, 3, 3, 3), F32, 305, 0.3),
        "conv_b": rand((4,), F32, 306, 0.1), "sm_x": rand((7, 33), F32, 307, 2.0),
        "pool_x": rand((2, 3, 8, 8), F16, 308), "row_x": np.arange(5, dtype=np.int32) * 7 - 3,
        "cat_a": rand((2, 3, 4), BF16, 309), "cat_b": rand((2, 5, 4), BF16, 310),
    }
    ins["mm_bt"] = synth.encode(np.ascontiguousarray(synth.decode(ins["mm_b"], BF16).T), BF16)
    for k, v in ins.items():
        np.ascontiguousarray(v).tofile(os.path.join(d, k + ".bin"))
    print(f"adapter_check {d}", flush=True)
    r = subprocess.run([CHECK, d], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout.split(), r.stdout + r.stderr
    lines = r.stdout.splitlines()
    assert lines[0] == "backend hip"

    def got(name, dt, shape):
        return np.fromfile(os.path.join(d, name + ".bin"), dtype=synth.storage_dtype(dt)).reshape(shape)

    mm = orc.matmul(ins["mm_a"], ins["mm_b"], BF16)
    assert_close(got("out_mm", BF16, (64, 80)), mm, BF16, what="adapter matmul")
    assert_close(got("out_mm_t", BF16, (64, 80)), mm, BF16, what="adapter matmul transB")
    assert_close(got("out_add", F16, (4, 5, 6)), orc.add(ins["add_a"], ins["add_b"], F16), F16, what="adapter add")
    assert_close(got("out_conv", F32, (2, 4, 9, 9)), orc.conv2d(ins["conv_x"], ins["conv_w"], ins["conv_b"], 1, 1, F32),
                 F32, what="adapter conv2d")
    assert_close(got("out_sm", F32, (7, 33)), orc.softmax(ins["sm_x"], F32), F32, what="adapter softmax")
    assert np.array_equal(got("out_pool", F16, (2, 3, 4, 4)), orc.max_pool2d(ins["pool_x"], 2, 2, 0, F16))
    assert np.array_equal(got("out_row", I32, (3, 5)), np.tile(ins["row_x"], (3, 1)))
    assert np.array_equal(got("out_cat", BF16, (2, 8, 4)), orc.concat([ins["cat_a"], ins["cat_b"]], 1, BF16))
    # the table MuNet's dispatch sees through the adapter is the library's
    names = {v: k for k, v in FEATURES.items()}
    rows = [ln.split()[1:] for ln in lines if ln.startswith("support ")]
    assert len(rows) == 13 * 4
    for f, dt, av, pol, acc in (map(int, r) for r in rows):
        s = query_support(names[f], dt)
        assert (bool(av), pol, acc) == (s.available, 0, s.preferred_accumulation_dtype), (f, dt)
    assert any(ln.startswith("training_only hip backend: relu_backward") for ln in lines)
