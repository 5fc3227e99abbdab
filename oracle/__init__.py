"""Parity oracle for the MI355X HIP backend -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker / the timed CPU
baseline. The product library never links or calls it.

Two interchangeable backends expose the same op API on host numpy storage
arrays (float32 for fp32, uint16 bit patterns for fp16/bf16, int32 ids):

* ``CpuOracle("restatement")`` -> ``oracle/libmunet_cpu_ref.so``, a C++
  restatement of MuNet's CPU-backend arithmetic (``munet_cpu_ref.cpp``).
* ``CpuOracle("reference")``   -> ``oracle/_ref/libmunet_ref.so``, MuNet's own
  CPU code compiled from /root/reference plus ``ref_driver.cpp``.

Model forwards composed from these ops live in ``oracle/models.py``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
RESTATEMENT_LIB = os.path.join(HERE, "libmunet_cpu_ref.so")
REFERENCE_LIB = os.path.join(HERE, "_ref", "libmunet_ref.so")

F32, F16, BF16, I32 = 0, 1, 2, 3
ADD, SUB, MUL, DIV = 0, 1, 2, 3

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _ints(vals):
    arr = (ctypes.c_int * max(1, len(vals)))(*[int(v) for v in vals])
    return arr


def storage_np(dt):
    return {F32: np.float32, F16: np.uint16, BF16: np.uint16, I32: np.int32}[dt]


def available(which="restatement"):
    return os.path.exists(RESTATEMENT_LIB if which == "restatement" else REFERENCE_LIB)


class OracleError(RuntimeError):
    pass


class CpuOracle:
    def __init__(self, which="restatement"):
        self.which = which
        path = RESTATEMENT_LIB if which == "restatement" else REFERENCE_LIB
        if not os.path.exists(path):
            raise FileNotFoundError(f"oracle library not built: {path} (run `make -C oracle`)")
        self.lib = ctypes.CDLL(path)
        self.pre = "orc_" if which == "restatement" else "ref_"
        getattr(self.lib, self.pre + "last_error").restype = ctypes.c_char_p

    def _call(self, name, *args):
        rc = getattr(self.lib, self.pre + name)(*args)
        if rc != 0:
            msg = getattr(self.lib, self.pre + "last_error")()
            raise OracleError(f"{self.which}.{name}: {msg.decode() if msg else rc}")

    def threads(self):
        """Threads the restatement's parallel loops use (hardware_concurrency)."""
        fn = getattr(self.lib, "orc_threads", None)
        return int(fn()) if fn else 1

    def set_threading(self, mode):
        """Restatement only. "parity": every loop over independent outputs is
        split over all hardware threads (fast checking). "reference": the
        reference's own split (CPUBackend::parallel_for, inline below 1024
        iterations, src/backend/cpu_backend.hpp:101-127; the typed fallbacks,
        LayerNorm, masked_fill and the gathers serial), for the timed CPU
        baseline. Results are bit-identical in both modes."""
        self._call("set_threading", _i({"parity": 0, "reference": 1}[mode]))

    @staticmethod
    def _c(a, dt):
        return np.ascontiguousarray(a, dtype=storage_np(dt))

    # -- codecs --------------------------------------------------------------
    def encode(self, x, dt):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, dtype=storage_np(dt))
        self._call("encode", _i(dt), _ptr(x), _ptr(out), _sz(x.size))
        return out

    def decode(self, s, dt):
        s = self._c(s, dt)
        out = np.empty(s.shape, dtype=np.float32)
        self._call("decode", _i(dt), _ptr(s), _ptr(out), _sz(s.size))
        return out

    # -- ops ---------------------------------------------------------------------
    def matmul(self, a, b, dt):
        """Tensor::matmul: a [M,K] or [batch..,M,K]; b [K,N] or [batch..,K,N]."""
        a, b = self._c(a, dt), self._c(b, dt)
        M, K, N = a.shape[-2], a.shape[-1], b.shape[-1]
        out = np.empty(a.shape[:-1] + (N,), dtype=storage_np(dt))
        if self.which == "reference":
            self._call("matmul", _i(dt), _ptr(a), _ints(a.shape), _i(a.ndim),
                       _ptr(b), _ints(b.shape), _i(b.ndim), _ptr(out))
        else:
            batch = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
            self._call("matmul", _i(dt), _ptr(a), _ptr(b), _ptr(out), _i(batch),
                       _i(M), _i(K), _i(N), _i(1 if b.ndim > 2 else 0), _i(0), _i(0))
        return out

    def binary(self, op, a, b, dt):
        a, b = self._c(a, dt), self._c(b, dt)
        oshape = np.broadcast_shapes(a.shape, b.shape)
        out = np.empty(oshape, dtype=storage_np(dt))
        self._call("binary", _i(dt), _i(op), _ptr(a), _ints(a.shape), _i(a.ndim),
                   _ptr(b), _ints(b.shape), _i(b.ndim), _ptr(out))
        return out

    def add(self, a, b, dt):
        return self.binary(ADD, a, b, dt)

    def sub(self, a, b, dt):
        return self.binary(SUB, a, b, dt)

    def mul(self, a, b, dt):
        return self.binary(MUL, a, b, dt)

    def div(self, a, b, dt):
        return self.binary(DIV, a, b, dt)

    def masked_fill(self, x, mask, value, dt):
        """ops::masked_fill (elementwise.cpp:8-53): mask int32, same shape as x;
        `value` is the double the op's ScalarValue carries."""
        x = self._c(x, dt)
        mask = np.ascontiguousarray(mask, dtype=np.int32)
        if mask.shape != x.shape:
            raise OracleError("masked_fill: input/mask shape mismatch")
        out = np.empty_like(x)
        self._call("masked_fill", _i(dt), _ptr(x), _ptr(mask), _ptr(out), _sz(x.size), ctypes.c_double(value))
        return out

    def _unary(self, name, x, dt):
        x = self._c(x, dt)
        out = np.empty_like(x)
        self._call(name, _i(dt), _ptr(x), _ptr(out), _sz(x.size))
        return out

    def relu(self, x, dt):
        return self._unary("relu", x, dt)

    def sigmoid(self, x, dt):
        return self._unary("sigmoid", x, dt)

    def gelu(self, x, dt):
        return self._unary("gelu", x, dt)

    def softmax(self, x, dt):
        x = self._c(x, dt)
        out = np.empty_like(x)
        cols = x.shape[-1]
        self._call("softmax", _i(dt), _ptr(x), _ptr(out), _i(x.size // cols), _i(cols))
        return out

    def layer_norm(self, x, w, b, dt, eps=1e-5):
        x, w, b = self._c(x, dt), self._c(w, dt), self._c(b, dt)
        out = np.empty_like(x)
        cols = x.shape[-1]
        self._call("layer_norm", _i(dt), _ptr(x), _ptr(w), _ptr(b), _ptr(out),
                   _i(x.size // cols), _i(cols), ctypes.c_float(eps))
        return out

    def linear(self, x, w, b, dt):
        """nn::Linear: y = x.matmul(W) + b (linear.hpp:28-34)."""
        if self.which == "reference":
            x, w = self._c(x, dt), self._c(w, dt)
            bb = None if b is None else self._c(b, dt)
            out = np.empty(x.shape[:-1] + (w.shape[1],), dtype=storage_np(dt))
            self._call("linear", _i(dt), _ptr(x), _ints(x.shape), _i(x.ndim), _ptr(w),
                       _ptr(bb), _i(w.shape[0]), _i(w.shape[1]), _ptr(out))
            return out
        y = self.matmul(x, w, dt)
        return y if b is None else self.add(y, b, dt)

    def mha(self, x, p, heads, causal, dt, prefix="", textbook=False):
        """nn::MultiHeadAttention forward on x [B,T,E]; p holds
        ``<prefix>{q,k,v,out}_proj.{weight,bias}``.  textbook: the attention
        core reads key j as position j's own key (mha_core)."""
        x = self._c(x, dt)
        B, T, E = x.shape
        g = lambda n: self._c(p[prefix + n], dt)
        if self.which == "reference":
            if textbook:
                raise ValueError("MuNet has no textbook-key attention")
            out = np.empty_like(x)
            self._call("mha", _i(dt), _ptr(x), _i(B), _i(T), _i(E), _i(heads), _i(int(causal)),
                       _ptr(g("q_proj.weight")), _ptr(g("q_proj.bias")),
                       _ptr(g("k_proj.weight")), _ptr(g("k_proj.bias")),
                       _ptr(g("v_proj.weight")), _ptr(g("v_proj.bias")),
                       _ptr(g("out_proj.weight")), _ptr(g("out_proj.bias")), _ptr(out))
            return out
        x2 = x.reshape(B * T, E)
        q = self.linear(x2, g("q_proj.weight"), g("q_proj.bias"), dt)
        k = self.linear(x2, g("k_proj.weight"), g("k_proj.bias"), dt)
        v = self.linear(x2, g("v_proj.weight"), g("v_proj.bias"), dt)
        ctx = self.mha_core(q, k, v, B, T, heads, causal, dt, textbook=textbook)
        return self.linear(ctx, g("out_proj.weight"), g("out_proj.bias"), dt).reshape(B, T, E)

    def mha_core(self, q2d, k2d, v2d, B, T, heads, causal, dt, textbook=False):
        """Restatement only: projected q/k/v [B*T,E] -> merged context [B*T,E].
        textbook=False: MuNet's reading of k's buffer as [hd, B*H*T]
        (src/nn/attention.hpp:64-67, src/core/ops/matmul.cpp:331-392);
        textbook=True: key j of a head is position j's key, with the same
        rounding steps (the build's decode attention; no MuNet counterpart)."""
        q2d, k2d, v2d = self._c(q2d, dt), self._c(k2d, dt), self._c(v2d, dt)
        out = np.empty_like(q2d)
        E = q2d.shape[-1]
        self._call("mha_core_textbook" if textbook else "mha_core", _i(dt), _ptr(q2d), _ptr(k2d), _ptr(v2d), _ptr(out),
                   _i(B), _i(T), _i(heads), _i(E // heads), _i(int(causal)))
        return out

    def embedding(self, ids, w, dt):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        w = self._c(w, dt)
        V, D = w.shape
        out = np.empty(ids.shape + (D,), dtype=storage_np(dt))
        if self.which == "reference":
            B, T = ids.shape
            self._call("embedding", _i(dt), _ptr(ids), _i(B), _i(T), _ptr(w), _i(V), _i(D), _ptr(out))
        else:
            self._call("embedding", _i(dt), _ptr(ids), _ptr(w), _ptr(out), _i(ids.size), _i(V), _i(D))
        return out

    def conv2d(self, x, w, b, stride, pad, dt):
        x, w = self._c(x, dt), self._c(w, dt)
        bb = None if b is None else self._c(b, dt)
        B, iC, iH, iW = x.shape
        oC, _, k, _ = w.shape
        oH, oW = (iH + 2 * pad - k) // stride + 1, (iW + 2 * pad - k) // stride + 1
        out = np.empty((B, oC, oH, oW), dtype=storage_np(dt))
        if self.which == "reference":
            self._call("conv2d", _i(dt), _ptr(x), _ptr(w), _ptr(bb), _ptr(out), _i(B), _i(iC),
                       _i(iH), _i(iW), _i(oC), _i(k), _i(stride), _i(pad))
        else:
            self._call("conv2d", _i(dt), _ptr(x), _ptr(w), _ptr(bb), _ptr(out), _i(B), _i(iC),
                       _i(iH), _i(iW), _i(oC), _i(k), _i(k), _i(stride), _i(pad))
        return out

    def max_pool2d(self, x, k, s, p, dt):
        x = self._c(x, dt)
        B, C, iH, iW = x.shape
        out = np.empty((B, C, (iH + 2 * p - k) // s + 1, (iW + 2 * p - k) // s + 1), dtype=storage_np(dt))
        self._call("max_pool2d", _i(dt), _ptr(x), _ptr(out), _i(B), _i(C), _i(iH), _i(iW), _i(k), _i(s), _i(p))
        return out

    def upsample2d(self, x, scale, dt):
        x = self._c(x, dt)
        B, C, iH, iW = x.shape
        out = np.empty((B, C, iH * scale, iW * scale), dtype=storage_np(dt))
        self._call("upsample2d", _i(dt), _ptr(x), _ptr(out), _i(B), _i(C), _i(iH), _i(iW), _i(scale))
        return out

    # -- MuNet's deploy-artifact loader (reference only) ---------------------
    def load_check(self, path):
        """None if MuNet's loader accepts the artifact at `path`, else its message."""
        rc = self.lib.ref_load_check(str(path).encode())
        return None if rc == 0 else self.lib.ref_last_error().decode()

    def load_forward(self, path, x, dt):
        """MuNet's loader on `path`, then the loaded module's forward on x."""
        x = self._c(x, dt)
        out = np.empty(64 << 20, dtype=np.uint8)
        shp = (ctypes.c_int * 8)()
        nd = ctypes.c_int()
        self._call("load_forward", ctypes.c_char_p(str(path).encode()), _i(dt), _ptr(x), _ints(x.shape), _i(x.ndim),
                   _ptr(out), _sz(out.nbytes), shp, ctypes.byref(nd))
        shape = tuple(shp[i] for i in range(nd.value))
        n = int(np.prod(shape)) * np.dtype(storage_np(dt)).itemsize
        return out[:n].view(storage_np(dt)).reshape(shape).copy()

    def concat(self, xs, dim, dt):
        xs = [self._c(x, dt) for x in xs]
        nd = xs[0].ndim
        oshape = list(xs[0].shape)
        oshape[dim] = sum(x.shape[dim] for x in xs)
        out = np.empty(oshape, dtype=storage_np(dt))
        ptrs = (_vp * len(xs))(*[x.ctypes.data for x in xs])
        shapes = _ints([d for x in xs for d in x.shape])
        self._call("concat", _i(dt), ptrs, shapes, _i(len(xs)), _i(nd), _i(dim), _ptr(out))
        return out
