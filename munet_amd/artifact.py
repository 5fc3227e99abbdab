"""Writer for MuNet deploy artifacts (``munet_model`` revision 1 .npz).

The format is the one the reference's loader reads
(src/inference_serialization.cpp:902-1080) and its writers produce
(src/bindings.cpp:2030-2062): an uncompressed .npz holding one array per
named parameter plus string / integer / boolean metadata scalars.  bf16
parameters, which the reference cannot store, are written as ``<u2`` arrays
of bf16 bit patterns (what ``mh_engine_create_from_artifact`` reads as bf16).
"""
from __future__ import annotations

import json

import numpy as np

from . import synth

FORMAT_NAME = "munet_model"
FORMAT_REVISION = 1


def _tensor(arr: np.ndarray, dtype: str) -> np.ndarray:
    a = np.ascontiguousarray(arr)
    if dtype == "float32":
        return a.astype(np.float32, copy=False)
    if dtype == "float16":  # storage bits -> IEEE binary16 array ('<f2')
        return a.view(np.float16) if a.dtype == np.uint16 else a.astype(np.float16)
    if dtype == "bfloat16":  # bf16 bit patterns ('<u2')
        if a.dtype != np.uint16:
            raise TypeError("bfloat16 parameters are given as uint16 bit patterns")
        return a
    if dtype == "int32":
        return a.astype(np.int32, copy=False)
    raise ValueError(f"unsupported dtype {dtype}")


def save_deploy_artifact(path: str, config: dict, params: dict, dtype: str | None = None) -> None:
    """Write `params` (storage format of `dtype`, default the config's) and
    `config` as a deploy artifact at `path`."""
    dtype = dtype or config.get("dtype", "float32")
    state = {name: _tensor(arr, dtype) for name, arr in params.items()}
    names = sorted(state)
    state.update({
        "__config__": np.array(json.dumps(config)),
        "__format_name__": np.array(FORMAT_NAME),
        "__format_revision__": np.array(FORMAT_REVISION, dtype=np.int64),
        "__format_version__": np.array("munet_model_v1"),
        "__producer__": np.array("munet"),
        "__artifact_kind__": np.array("deploy_model"),
        "__artifact_scope__": np.array("runtime_only"),
        "__default_load_mode__": np.array("eval"),
        "__contains_training_state__": np.array(False),
        "__recommended_loader__": np.array("load_for_inference"),
        "__compile_contract_policy__": np.array("external"),
        "__device_policy__": np.array("caller_specified"),
        "__dtype_policy__": np.array("per_tensor"),
        "__tensor_names__": np.array(json.dumps(names)),
    })
    with open(path, "wb") as f:
        np.savez(f, **state)


def decode_params(params: dict, dtype: str) -> dict:
    """Float32 copies of storage-format parameters (for cross-dtype tests)."""
    dt = synth.DTYPE_CODES[dtype]
    return {k: synth.decode(v, dt) for k, v in params.items()}
