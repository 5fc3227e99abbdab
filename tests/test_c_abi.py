"""The C ABI libraries load and export every symbol their headers declare
(no compute call: runs without a GPU)."""
import ctypes
import os
import re

import pytest

from munet_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:mh|munet_backend_plugin)_\w+)\s*\(", text)))


@pytest.mark.parametrize("header", ["munet_hip.h", "munet_hip_engine.h"])
def test_library_exports_every_declared_symbol(header):
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = _declared(header)
    assert len(names) > 5
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{header}: not exported: {missing}"


def test_python_binding_covers_header():
    names = set(_declared("munet_hip.h") + _declared("munet_hip_engine.h"))
    bound = set(_lib.exported_symbols())
    assert not (names - bound), sorted(names - bound)


def test_plugin_probe_abi():
    """MuNet's plugin loader contract (reference src/backend/plugin_loader.cpp:122-131)."""
    lib = ctypes.CDLL(_lib.PLUGIN_PATH)
    lib.munet_backend_plugin_abi_version.restype = ctypes.c_uint32
    lib.munet_backend_plugin_name.restype = ctypes.c_char_p
    lib.munet_backend_plugin_device_type.restype = ctypes.c_char_p
    lib.munet_backend_plugin_probe.restype = ctypes.c_char_p
    lib.munet_backend_plugin_capability_flags.restype = ctypes.c_uint64
    assert lib.munet_backend_plugin_abi_version() == 1
    assert lib.munet_backend_plugin_name() == b"hip"
    assert lib.munet_backend_plugin_device_type() == b"hip"
    assert lib.munet_backend_plugin_capability_flags() & 0x7
    # the probe returns nullptr (usable) or a reason string; both are valid here
    r = lib.munet_backend_plugin_probe()
    assert r is None or isinstance(r, bytes)


def test_error_reporting_without_gpu():
    """Invalid arguments fail with a message instead of touching the device."""
    with pytest.raises(_lib.HipError, match="unsupported dtype"):
        _lib.call("mh_relu", 7, None, None, 0, None)
