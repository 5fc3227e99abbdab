"""ctypes binding of libmunet_hip.so (C ABI in include/munet_hip.h).

The library is built in-tree by ``munet_amd.build``.  Loading fails loudly
when it is missing: there is no CPU or PyTorch fallback for any op.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmunet_hip.so")
PLUGIN_PATH = os.path.join(HERE, "libmunet_backend_hip.so")

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_i64 = ctypes.c_int64
_f = ctypes.c_float
_d = ctypes.c_double
_ip = ctypes.POINTER(ctypes.c_int)
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes (all return int status unless listed in _RESTYPES)
_SIGS = {
    "mh_device_count": [_ip],
    "mh_init": [_i],
    "mh_check_device_errors": [],
    "mh_allocate": [ctypes.POINTER(_vp), _sz],
    "mh_deallocate": [_vp],
    "mh_memset": [_vp, _i, _sz, _vp],
    "mh_copy": [_vp, _vp, _sz, _i, _i, _vp],
    "mh_synchronize": [_vp],
    "mh_to_contiguous": [_i, _vp, _vp, _i, _ip, _i64p, _i64, _vp],
    "mh_add": [_i, _vp, _vp, _vp, _i, _ip, _i64p, _i64p, _vp],
    "mh_sub": [_i, _vp, _vp, _vp, _i, _ip, _i64p, _i64p, _vp],
    "mh_mul": [_i, _vp, _vp, _vp, _i, _ip, _i64p, _i64p, _vp],
    "mh_div": [_i, _vp, _vp, _vp, _i, _ip, _i64p, _i64p, _vp],
    "mh_relu": [_i, _vp, _vp, _sz, _vp],
    "mh_sigmoid": [_i, _vp, _vp, _sz, _vp],
    "mh_exp": [_i, _vp, _vp, _sz, _vp],
    "mh_log": [_i, _vp, _vp, _sz, _vp],
    "mh_sqrt": [_i, _vp, _vp, _sz, _vp],
    "mh_rsqrt": [_i, _vp, _vp, _sz, _vp],
    "mh_sin": [_i, _vp, _vp, _sz, _vp],
    "mh_cos": [_i, _vp, _vp, _sz, _vp],
    "mh_gelu": [_i, _vp, _vp, _sz, _vp],
    "mh_softmax": [_i, _vp, _vp, _i, _i, _vp],
    "mh_masked_fill": [_i, _vp, _vp, _vp, _sz, _d, _vp],
    "mh_layer_norm": [_i, _vp, _vp, _vp, _vp, _i, _i, _f, _vp],
    "mh_embedding": [_i, _vp, _vp, _vp, _i, _i, _i, _vp],
    "mh_embedding_pos": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "mh_convert": [_i, _vp, _i, _vp, _sz, _vp],
    "mh_check_f16_rounding": [ctypes.POINTER(ctypes.c_ulonglong), _vp],
    "mh_argmax": [_i, _vp, _vp, _i, _i, _vp],
    "mh_measure_mfma_peak": [_i, _i, ctypes.POINTER(ctypes.c_double), _vp],
    "mh_measure_hbm_read": [_vp, _sz, _i, ctypes.POINTER(ctypes.c_double), _vp],
    "mh_query_support": [_i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "mh_matmul": [_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "mh_matmul_noalloc": [_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "mh_batched_matmul": [_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i64, _i64, _i64, _vp],
    "mh_linear": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp],
    "mh_pack_linear_weight": [_i, _vp, _vp, _i, _i, _vp],
    "mh_qkv_projection": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "mh_attention": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "mh_attention_textbook": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "mh_concat": [_i, ctypes.POINTER(_vp), _i, _vp, _i, _i, _ip, _vp],
    "mh_transpose2d": [_i, _vp, _vp, _i, _i, _i, _vp],
    "mh_conv2d": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp],
    "mh_conv2d_nhwc": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp],
    "mh_pack_conv_weight": [_i, _vp, _vp, _i, _i, _i, _i, _vp],
    "mh_conv_transpose2d_nhwc": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i64, _vp],
    "mh_pack_convt_weight": [_i, _vp, _vp, _i, _i, _i, _vp],
    "mh_max_pool2d": [_i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp],
    "mh_max_pool2d_nhwc": [_i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp],
    "mh_upsample2d": [_i, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "mh_upsample2d_nhwc": [_i, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "mh_nchw_to_nhwc": [_i, _vp, _vp, _i, _i, _i, _vp],
    "mh_nhwc_to_nchw": [_i, _vp, _vp, _i, _i, _i, _vp],
    # engine (include/munet_hip_engine.h)
    "mh_engine_create": [ctypes.POINTER(_vp), ctypes.c_char_p, _i],
    "mh_engine_destroy": [_vp],
    "mh_engine_create_from_artifact": [ctypes.POINTER(_vp), ctypes.c_char_p, _i],
    "mh_engine_set_param": [_vp, ctypes.c_char_p, _vp, _sz, _i],
    "mh_engine_load": [_vp],
    "mh_engine_set_config": [_vp, _i, _i, _i],
    "mh_engine_compile": [_vp, _ip, _i],
    "mh_engine_input_ptr": [_vp, ctypes.POINTER(_vp)],
    "mh_engine_output_ptr": [_vp, ctypes.POINTER(_vp)],
    "mh_engine_output_shape": [_vp, _ip, _ip],
    "mh_engine_run": [_vp, _vp, _vp],
    "mh_engine_run_device": [_vp],
    "mh_engine_launch": [_vp],
    "mh_engine_stats": [_vp, ctypes.c_char_p, _sz],
    "mh_engine_plan": [_vp, ctypes.c_char_p, _sz],
    "mh_engine_op_times": [_vp, ctypes.c_int, ctypes.c_char_p, ctypes.c_char_p, _sz],
    "mh_engine_forward_op_times": [_vp, ctypes.c_int, ctypes.c_char_p, _sz],
    "mh_decoder_create": [ctypes.POINTER(_vp), _vp, _i, _i],
    "mh_decoder_destroy": [_vp],
    "mh_decoder_prefill": [_vp, _vp, _i, _vp],
    "mh_decoder_step": [_vp, _vp, _vp, _vp],
    "mh_decoder_generate": [_vp, _i, _vp, ctypes.POINTER(ctypes.c_float)],
    "mh_decoder_position": [_vp, ctypes.POINTER(_i)],
    "mh_decoder_stats": [_vp, ctypes.c_char_p, _sz],
    "mh_engine_stream": [_vp, ctypes.POINTER(_vp)],
    "mh_engine_compile_expected": [_vp, _ip, _i, _ip],
    "mh_engine_output_shape_for": [_vp, _ip, _i, _ip, _ip],
    "mh_engine_run_shaped": [_vp, _vp, _ip, _i, _vp],
    "mh_engine_run_cached": [_vp, _vp, ctypes.c_uint64, ctypes.c_uint64, _vp],
    "mh_engine_set_input_cache": [_vp, _sz, _sz],
    "mh_engine_clear_input_cache": [_vp],
    "mh_engine_run_batch": [_vp, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp)],
    "mh_engine_set_observer": [_vp, _vp, _vp],
    "mh_engine_pinned_io": [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp)],
    "mh_engine_run_pinned": [_vp],
}
_RESTYPES = {
    "mh_last_error": ctypes.c_char_p,
    "mh_version": ctypes.c_char_p,
    "mh_get_last_kernel_time_us": ctypes.c_double,
}

_lock = threading.Lock()
_lib = None


class HipError(RuntimeError):
    """A libmunet_hip.so call failed (MuNet backends raise std::runtime_error)."""


def exported_symbols():
    return sorted(list(_SIGS) + list(_RESTYPES))


def load():
    """Load libmunet_hip.so (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP backend with `python -m munet_amd.build` "
                "(there is no CPU fallback)")
        # One HIP runtime per process: torch ships its own libamdhip64 (same
        # SONAME, different file).  Loading torch first makes this library's
        # NEEDED libamdhip64.so.7 bind to the runtime torch already loaded;
        # the other order would start a second HIP/HSA runtime in the process.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = ctypes.CDLL(LIB_PATH)
        for name, argt in _SIGS.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.argtypes = argt
            fn.restype = ctypes.c_int
        for name, rt in _RESTYPES.items():
            fn = getattr(lib, name)
            fn.restype = rt
            fn.argtypes = []
        _lib = lib
        return lib


def call(name, *args):
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.mh_last_error()
        raise HipError(f"{name}: {msg.decode() if msg else rc}")
    return rc


def ints(vals):
    vals = [int(v) for v in vals]
    return (ctypes.c_int * max(1, len(vals)))(*vals)


def i64s(vals):
    vals = [int(v) for v in vals]
    return (ctypes.c_int64 * max(1, len(vals)))(*vals)
