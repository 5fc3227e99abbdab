"""Python mirror of MuNet's ``Backend`` capability interface for the HIP backend.

Method names, argument order and meaning follow the reference's capability
classes (src/core/backend.hpp:190-345); a ``Storage`` here is any torch
tensor living on the GPU (torch only provides device memory and the stream),
and every compute call goes through libmunet_hip.so.  Errors raise
``HipError`` as MuNet's backends raise std::runtime_error.

``query_support`` mirrors Backend::query_support (src/core/backend.hpp:
411-425): fp32/fp16/bf16 are available for every implemented feature and
the fallback policy is always ExplicitUnsupported - this backend never
falls back to the CPU.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import call, i64s, ints
from .synth import BF16, F16, F32, I32

_vp = ctypes.c_void_p


def _torch():
    import torch
    return torch


def torch_dtype(dt):
    t = _torch()
    return {F32: t.float32, F16: t.float16, BF16: t.bfloat16, I32: t.int32}[dt]


def dtype_code(tdtype):
    t = _torch()
    return {t.float32: F32, t.float16: F16, t.bfloat16: BF16, t.int32: I32}[tdtype]


def to_device(arr: np.ndarray, dt: int, device="cuda"):
    """Host storage array (float32 / uint16 bits / int32) -> GPU tensor with the same bits."""
    t = _torch()
    a = np.ascontiguousarray(arr)
    if dt in (F16, BF16):
        host = t.from_numpy(a.astype(np.uint16, copy=False).view(np.int16)).view(torch_dtype(dt))
    elif dt == F32:
        host = t.from_numpy(a.astype(np.float32, copy=False))
    else:
        host = t.from_numpy(a.astype(np.int32, copy=False))
    return host.to(device)


def to_host(x, dt: int) -> np.ndarray:
    """GPU tensor -> host storage array (uint16 bit patterns for 16-bit types)."""
    t = _torch()
    c = x.detach().contiguous().cpu()
    if dt in (F16, BF16):
        return c.view(t.int16).numpy().view(np.uint16).copy()
    return c.numpy().copy()


def empty(shape, dt, device="cuda"):
    return _torch().empty(tuple(shape), dtype=torch_dtype(dt), device=device)


def _p(x):
    return None if x is None else _vp(x.data_ptr())


def _stream():
    return _vp(_torch().cuda.current_stream().cuda_stream)


def _dt(x):
    return dtype_code(x.dtype)


def compute_broadcast(a_shape, a_strides, b_shape, b_strides):
    """compute_broadcast (reference src/types.hpp:436-478)."""
    nd = max(len(a_shape), len(b_shape))
    out, sa, sb = [1] * nd, [0] * nd, [0] * nd
    for i in range(nd):
        ia, ib, o = len(a_shape) - 1 - i, len(b_shape) - 1 - i, nd - 1 - i
        da = a_shape[ia] if ia >= 0 else 1
        db = b_shape[ib] if ib >= 0 else 1
        if da != db and da != 1 and db != 1:
            raise ValueError(f"shape mismatch {tuple(a_shape)} vs {tuple(b_shape)}")
        out[o] = max(da, db)
        sa[o] = (0 if (da == 1 and db != 1) else a_strides[ia]) if ia >= 0 else 0
        sb[o] = (0 if (db == 1 and da != 1) else b_strides[ib]) if ib >= 0 else 0
    return out, sa, sb


def contiguous_strides(shape):
    s, out = 1, []
    for d in reversed(shape):
        out.append(s)
        s *= d
    return list(reversed(out))


@dataclass
class BroadcastInfo:
    out_shape: list
    strides_a: list
    strides_b: list


@dataclass
class BackendSupport:
    available: bool
    fallback_policy: str
    preferred_accumulation_dtype: int


# BackendFeature (reference src/core/backend.hpp:16-30, in its order) and the
# path's functions that have no reference capability: the mh_query_support codes
FEATURES = {"elementwise_binary": 0, "broadcast_row": 1, "matmul": 2, "unary_activation": 3, "softmax": 4,
            "concat": 5, "loss": 6, "convolution": 7, "pooling": 8, "batch_norm": 9, "optimizer_step": 10,
            "random_fill": 11, "reduction": 12, "to_contiguous": 100, "layer_norm": 101, "attention": 102,
            "embedding": 103, "masked_fill": 104}
POLICIES = ("ExplicitUnsupported", "CPUFallback", "ConversionFallback")


def query_support(feature: str, dtype: int) -> BackendSupport:
    """Backend::query_support (src/core/backend.hpp:411-425) of the HIP
    backend, from mh_query_support (no device needed). Unknown features are
    unavailable."""
    av, pol, acc = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    call("mh_query_support", FEATURES.get(feature, -1), dtype, ctypes.byref(av), ctypes.byref(pol),
         ctypes.byref(acc))
    return BackendSupport(bool(av.value), POLICIES[pol.value], acc.value)


class HipBackend:
    """The HIP backend's capability surface (reference class Backend)."""

    def __init__(self, device: int = 0):
        self.device = device
        call("mh_init", device)

    def name(self):
        return "hip"

    def query_support(self, feature: str, dtype: int, shape=None) -> BackendSupport:
        return query_support(feature, dtype)

    # ---- allocation / transfer (backend.hpp:190-205) ----------------------
    def allocate(self, nbytes: int) -> int:
        p = _vp()
        call("mh_allocate", ctypes.byref(p), nbytes)
        return p.value or 0

    def deallocate(self, ptr: int):
        call("mh_deallocate", _vp(ptr))

    def memset(self, x, value: int, nbytes: int):
        call("mh_memset", _p(x), value, nbytes, _stream())

    def synchronize(self):
        call("mh_synchronize", _stream())

    def get_last_kernel_time_us(self) -> float:
        return _lib.load().mh_get_last_kernel_time_us()

    def reports_gpu_kernel_time(self) -> bool:
        return True

    def to_contiguous(self, src, dst, shape, strides, offset=0):
        call("mh_to_contiguous", _dt(src), _p(src), _p(dst), len(shape), ints(shape), i64s(strides), offset,
             _stream())

    # ---- elementwise (backend.hpp:207-238) --------------------------------
    def _bin(self, name, a, b, out, info: BroadcastInfo):
        call(name, _dt(a), _p(a), _p(b), _p(out), len(info.out_shape), ints(info.out_shape), i64s(info.strides_a),
             i64s(info.strides_b), _stream())

    def add(self, a, b, out, info):
        self._bin("mh_add", a, b, out, info)

    def sub(self, a, b, out, info):
        self._bin("mh_sub", a, b, out, info)

    def mul(self, a, b, out, info):
        self._bin("mh_mul", a, b, out, info)

    def div(self, a, b, out, info):
        self._bin("mh_div", a, b, out, info)

    def _un(self, name, x, out, n):
        call(name, _dt(x), _p(x), _p(out), n, _stream())

    def relu(self, x, out, n):
        self._un("mh_relu", x, out, n)

    def sigmoid(self, x, out, n):
        self._un("mh_sigmoid", x, out, n)

    def exp(self, x, out, n):
        self._un("mh_exp", x, out, n)

    def log(self, x, out, n):
        self._un("mh_log", x, out, n)

    def sqrt(self, x, out, n):
        self._un("mh_sqrt", x, out, n)

    def rsqrt(self, x, out, n):
        self._un("mh_rsqrt", x, out, n)

    def sin(self, x, out, n):
        self._un("mh_sin", x, out, n)

    def cos(self, x, out, n):
        self._un("mh_cos", x, out, n)

    def softmax(self, x, out, batch_size, num_classes):
        call("mh_softmax", _dt(x), _p(x), _p(out), batch_size, num_classes, _stream())

    # ---- op-layer functions without a reference backend hook ---------------
    def gelu(self, x, out, n):
        self._un("mh_gelu", x, out, n)

    def masked_fill(self, x, mask, out, n, value):
        call("mh_masked_fill", _dt(x), _p(x), _p(mask), _p(out), n, float(value), _stream())

    def layer_norm(self, x, w, b, out, rows, cols, eps=1e-5):
        call("mh_layer_norm", _dt(x), _p(x), _p(w), _p(b), _p(out), rows, cols, eps, _stream())

    def embedding(self, ids, w, out, n, V, D):
        call("mh_embedding", _dt(w), _p(ids), _p(w), _p(out), n, V, D, _stream())

    def embedding_pos(self, ids, tok_w, pos_w, out, n, V, D, T):
        call("mh_embedding_pos", _dt(tok_w), _p(ids), _p(tok_w), _p(pos_w), _p(out), n, V, D, T, _stream())

    def check_device_errors(self):
        call("mh_check_device_errors")

    def convert(self, x, out, n):
        call("mh_convert", _dt(x), _p(x), _dt(out), _p(out), n, _stream())

    def check_f16_rounding(self) -> int:
        """Float bit patterns (of all 2^32) where the kernels' fast fp16
        rounding differs from the full codec (no reference counterpart)."""
        n = ctypes.c_ulonglong(0)
        call("mh_check_f16_rounding", ctypes.byref(n), _stream())
        return n.value

    def argmax(self, x, out, rows, cols):
        call("mh_argmax", _dt(x), _p(x), _p(out), rows, cols, _stream())

    def measure_mfma_peak(self, dt=2, iters=16000) -> float:
        """Measured matrix-core peak in FLOP/s (mh_measure_mfma_peak; dt 2 =
        bf16, 1 = fp16) on the current torch stream."""
        v = ctypes.c_double(0.0)
        call("mh_measure_mfma_peak", dt, iters, ctypes.byref(v), _stream())
        return v.value

    def measure_hbm_read(self, buf, reps=5) -> float:
        """Measured HBM read rate in bytes/s over the device tensor ``buf``
        (mh_measure_hbm_read)."""
        v = ctypes.c_double()
        call("mh_measure_hbm_read", _p(buf), buf.numel() * buf.element_size(), reps, ctypes.byref(v), _stream())
        return v.value

    # ---- blas (backend.hpp:250-260) ----------------------------------------
    def matmul(self, a, b, out, M, K, N, transA=False, transB=False):
        call("mh_matmul", _dt(a), _p(a), _p(b), _p(out), M, K, N, int(transA), int(transB), _stream())

    def matmul_noalloc(self, a, b, out, M, K, N, transA=False, transB=False):
        """mh_matmul_noalloc: mh_matmul staging its transposes in the
        library's fixed per-device scratch (no device allocation)."""
        call("mh_matmul_noalloc", _dt(a), _p(a), _p(b), _p(out), M, K, N, int(transA), int(transB), _stream())

    def batched_matmul(self, a, b, out, batch, M, K, N, transA, transB, stride_a, stride_b, stride_out):
        call("mh_batched_matmul", _dt(a), _p(a), _p(b), _p(out), batch, M, K, N, int(transA), int(transB),
             stride_a, stride_b, stride_out, _stream())

    def pack_linear_weight(self, w, w_t, in_f, out_f):
        call("mh_pack_linear_weight", _dt(w), _p(w), _p(w_t), in_f, out_f, _stream())

    def linear(self, x, w_t, bias, out, M, K, N, act=0, resid=None):
        call("mh_linear", _dt(x), _p(x), _p(w_t), _p(bias), _p(out), M, K, N, act, _p(resid), _stream())

    def qkv_projection(self, x, wqkv_t, bqkv, q, k, v, B, T, E, H):
        call("mh_qkv_projection", _dt(x), _p(x), _p(wqkv_t), _p(bqkv), _p(q), _p(k), _p(v), B, T, E, H,
             _stream())

    def attention(self, q, k, v, ctx, B, H, T, hd, causal):
        call("mh_attention", _dt(q), _p(q), _p(k), _p(v), _p(ctx), B, H, T, hd, int(causal), _stream())

    def attention_textbook(self, q, k, v, ctx, B, H, T, hd, causal):
        """Textbook keys (key j of a head is row j of its k): the decode
        attention; no MuNet counterpart."""
        call("mh_attention_textbook", _dt(q), _p(q), _p(k), _p(v), _p(ctx), B, H, T, hd, int(causal), _stream())

    # ---- shape (backend.hpp:263-271) ---------------------------------------
    def concat(self, inputs, out, dim, shapes):
        ptrs = (_vp * len(inputs))(*[x.data_ptr() for x in inputs])
        flat = [d for s in shapes for d in s]
        call("mh_concat", _dt(out), ptrs, len(inputs), _p(out), dim, len(shapes[0]), ints(flat), _stream())

    def transpose2d(self, x, out, batch, rows, cols):
        call("mh_transpose2d", _dt(x), _p(x), _p(out), batch, rows, cols, _stream())

    # ---- spatial (backend.hpp:291-311) -------------------------------------
    def conv2d(self, x, w, bias, out, B, iC, iH, iW, oC, kH, kW, s, p):
        call("mh_conv2d", _dt(x), _p(x), _p(w), _p(bias), _p(out), B, iC, iH, iW, oC, kH, kW, s, p, _stream())

    def conv2d_nhwc(self, x, w_ohwi, bias, out, B, iC, iH, iW, oC, kH, kW, s, p, act=0):
        call("mh_conv2d_nhwc", _dt(x), _p(x), _p(w_ohwi), _p(bias), _p(out), B, iC, iH, iW, oC, kH, kW, s, p, act,
             _stream())

    def pack_conv_weight(self, w, w_ohwi, oC, iC, kH, kW):
        call("mh_pack_conv_weight", _dt(w), _p(w), _p(w_ohwi), oC, iC, kH, kW, _stream())

    def conv_transpose2d_nhwc(self, x, w_packed, bias, out, B, iC, iH, iW, oC, k, ldc=None):
        call("mh_conv_transpose2d_nhwc", _dt(x), _p(x), _p(w_packed), _p(bias), _p(out), B, iC, iH, iW, oC, k,
             oC if ldc is None else ldc, _stream())

    def pack_convt_weight(self, w, w_packed, iC, oC, k):
        call("mh_pack_convt_weight", _dt(w), _p(w), _p(w_packed), iC, oC, k, _stream())

    def max_pool2d(self, x, out, B, C, iH, iW, k, s, p):
        call("mh_max_pool2d", _dt(x), _p(x), _p(out), B, C, iH, iW, k, s, p, _stream())

    def max_pool2d_nhwc(self, x, out, B, C, iH, iW, k, s, p):
        call("mh_max_pool2d_nhwc", _dt(x), _p(x), _p(out), B, C, iH, iW, k, s, p, _stream())

    def upsample2d(self, x, out, B, C, iH, iW, scale):
        call("mh_upsample2d", _dt(x), _p(x), _p(out), B, C, iH, iW, scale, _stream())

    def upsample2d_nhwc(self, x, out, B, C, iH, iW, scale):
        call("mh_upsample2d_nhwc", _dt(x), _p(x), _p(out), B, C, iH, iW, scale, _stream())

    def nchw_to_nhwc(self, x, out, B, C, HW):
        call("mh_nchw_to_nhwc", _dt(x), _p(x), _p(out), B, C, HW, _stream())

    def nhwc_to_nchw(self, x, out, B, C, HW):
        call("mh_nhwc_to_nchw", _dt(x), _p(x), _p(out), B, C, HW, _stream())
