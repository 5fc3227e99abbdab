"""Engine: the compiled HIP executor behind MuNet's inference::Engine contract.

Mirrors ``inference::Engine`` (reference src/inference.hpp:292-801):

* ``Engine.load(config, params)`` - module config in the reference's
  serialized schema (src/inference_serialization.cpp:762-860) and parameters
  by ``named_parameters`` name (src/core/module.hpp:95-107);
* ``Engine.load_artifact(path)`` - the same from a MuNet deploy artifact
  (``munet_model`` rev-1 .npz, reference inference::load_serialized,
  src/inference_serialization.cpp:902-1080), parsed and validated in
  libmunet_hip.so;
* ``compile(example_input)`` - exact shape contract; traces, fuses, plans the
  arena and captures the forward as a hipGraph (src/inference.hpp:446-537);
* ``run(x)`` - host input in storage format -> host output
  (src/inference.hpp:541-610); ``run_device()`` forwards on the resident
  input buffer (used by the benchmark, inputs already in HBM);
* ``stats()`` - EngineStats fields (src/inference.hpp:43-66) plus the
  executor's own (arena bytes, fused epilogues, ops).

All compute runs in libmunet_hip.so; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _lib, synth

_vp = ctypes.c_void_p


class Engine:
    def __init__(self, device: int = 0):
        self.device = device
        self._h = None
        self.config = None
        self.out_shape = None
        self.in_shape = None

    # -- load ---------------------------------------------------------------
    def load(self, config: dict, params: dict):
        lib = _lib.load()
        h = _vp()
        _lib.call("mh_engine_create", ctypes.byref(h), json.dumps(config).encode(), self.device)
        self._h = h
        self.config = config
        dt = synth.DTYPE_CODES[config.get("dtype", "float32")]
        for name, arr in params.items():
            a = np.ascontiguousarray(arr)
            # the storage dtype of each array: float32 and float16 values, uint16
            # bit patterns of the model's 16-bit dtype, int32; the engine converts
            # another floating dtype with MuNet's codecs and rejects the rest
            if a.dtype == np.float16:
                a, pdt = a.view(np.uint16), synth.F16
            elif a.dtype == np.uint16:
                pdt = dt if dt in (synth.F16, synth.BF16) else synth.BF16
            else:
                pdt = {np.dtype(np.float32): synth.F32, np.dtype(np.int32): synth.I32}.get(a.dtype)
                if pdt is None:
                    raise TypeError(f"parameter '{name}': unsupported array dtype {a.dtype}")
            _lib.call("mh_engine_set_param", h, name.encode(), a.ctypes.data_as(_vp), a.nbytes, pdt)
        del lib
        return self

    def finish_load(self):
        """Engine::load's completion: emits LoadStarted / LoadCompleted to the
        observer (compile does it otherwise)."""
        _lib.call("mh_engine_load", self._h)
        return self

    def set_config(self, warmup_runs: int = 0, strict_shape_check: bool = True, lean_mode: bool = False):
        """EngineConfig (reference src/inference.hpp:32-41)."""
        _lib.call("mh_engine_set_config", self._h, int(warmup_runs), int(bool(strict_shape_check)), int(bool(lean_mode)))
        self.strict = bool(strict_shape_check)
        return self

    def load_artifact(self, path: str):
        h = _vp()
        _lib.call("mh_engine_create_from_artifact", ctypes.byref(h), str(path).encode(), self.device)
        self._h = h
        # the config is read again here only for the output dtype on the host
        with np.load(path, allow_pickle=False) as z:
            self.config = json.loads(str(z["__config__"]))
        return self

    # -- compile ------------------------------------------------------------
    def compile(self, example_input_shape, expected_input_shape=None):
        """Exact shape contract, or `expected_input_shape` with -1 wildcards:
        other shapes meeting it get their own compiled instance on first run."""
        shape = [int(s) for s in example_input_shape]
        if expected_input_shape is None:
            _lib.call("mh_engine_compile", self._h, _lib.ints(shape), len(shape))
        else:
            exp = [int(s) for s in expected_input_shape]
            if len(exp) != len(shape):
                raise ValueError("expected_input_shape rank differs from the example's")
            _lib.call("mh_engine_compile_expected", self._h, _lib.ints(shape), len(shape), _lib.ints(exp))
        self.expected = None if expected_input_shape is None else tuple(int(s) for s in expected_input_shape)
        self.in_shape = tuple(shape)
        dims = (ctypes.c_int * 8)()
        nd = ctypes.c_int()
        _lib.call("mh_engine_output_shape", self._h, dims, ctypes.byref(nd))
        self.out_shape = tuple(dims[i] for i in range(nd.value))
        return self

    # -- run ----------------------------------------------------------------
    def _out_dtype(self):
        return synth.storage_dtype(synth.DTYPE_CODES[self.config.get("dtype", "float32")])

    def output_shape_for(self, input_shape) -> tuple:
        shape = [int(s) for s in input_shape]
        dims = (ctypes.c_int * 8)()
        nd = ctypes.c_int()
        _lib.call("mh_engine_output_shape_for", self._h, _lib.ints(shape), len(shape), dims, ctypes.byref(nd))
        return tuple(dims[i] for i in range(nd.value))

    def run(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x)
        if tuple(x.shape) == self.in_shape:
            out = np.empty(self.out_shape, dtype=self._out_dtype())
            _lib.call("mh_engine_run", self._h, x.ctypes.data_as(_vp), out.ctypes.data_as(_vp))
            return out
        if getattr(self, "expected", None) is None and getattr(self, "strict", True):
            raise ValueError(f"input shape {tuple(x.shape)} does not match the compiled contract {self.in_shape}")
        out = np.empty(self.output_shape_for(x.shape), dtype=self._out_dtype())
        _lib.call("mh_engine_run_shaped", self._h, x.ctypes.data_as(_vp), _lib.ints(x.shape), x.ndim,
                  out.ctypes.data_as(_vp))
        return out

    def run_prepared(self, x: np.ndarray, key: int, version: int = 0) -> np.ndarray:
        """Run through the prepared-input cache: `key` names the caller's input
        tensor, `version` its mutation count (reference prepare_input)."""
        x = np.ascontiguousarray(x)
        if tuple(x.shape) != self.in_shape:
            raise ValueError(f"input shape {tuple(x.shape)} does not match the compiled contract {self.in_shape}")
        out = np.empty(self.out_shape, dtype=self._out_dtype())
        _lib.call("mh_engine_run_cached", self._h, x.ctypes.data_as(_vp), int(key), int(version),
                  out.ctypes.data_as(_vp))
        return out

    def set_input_cache(self, max_entries: int, max_bytes: int):
        _lib.call("mh_engine_set_input_cache", self._h, int(max_entries), int(max_bytes))

    def clear_input_cache(self):
        _lib.call("mh_engine_clear_input_cache", self._h)

    def run_batch(self, xs) -> list:
        """run_batch_into: one forward per input, in order."""
        xs = [np.ascontiguousarray(x) for x in xs]
        for x in xs:
            if tuple(x.shape) != self.in_shape:
                raise ValueError(f"input shape {tuple(x.shape)} does not match the compiled contract {self.in_shape}")
        outs = [np.empty(self.out_shape, dtype=self._out_dtype()) for _ in xs]
        ins = (_vp * max(1, len(xs)))(*[x.ctypes.data for x in xs])
        os_ = (_vp * max(1, len(outs)))(*[o.ctypes.data for o in outs])
        _lib.call("mh_engine_run_batch", self._h, len(xs), ins, os_)
        return outs

    _OBSERVER = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_void_p)

    def set_observer(self, fn):
        """fn(event: dict) for each engine event (None removes it)."""
        if fn is None:
            self._observer = None
            _lib.call("mh_engine_set_observer", self._h, None, None)
            return
        self._observer = self._OBSERVER(lambda ev, _user: fn(json.loads(ev.decode())))
        _lib.call("mh_engine_set_observer", self._h, ctypes.cast(self._observer, _vp), None)

    def pinned_io(self):
        """(input, output) numpy views of the engine's page-locked staging
        buffers; fill the input, call run_pinned(), read the output."""
        pi, po = _vp(), _vp()
        _lib.call("mh_engine_pinned_io", self._h, ctypes.byref(pi), ctypes.byref(po))
        in_dt = np.int32 if self.config.get("type") in ("DecoderLM", "Embedding") else self._out_dtype()
        n_in = int(np.prod(self.in_shape)) * np.dtype(in_dt).itemsize
        n_out = int(np.prod(self.out_shape)) * np.dtype(self._out_dtype()).itemsize
        a = np.ctypeslib.as_array((ctypes.c_uint8 * n_in).from_address(pi.value)).view(in_dt).reshape(self.in_shape)
        b = np.ctypeslib.as_array((ctypes.c_uint8 * n_out).from_address(po.value)).view(self._out_dtype())
        return a, b.reshape(self.out_shape)

    def run_pinned(self):
        _lib.call("mh_engine_run_pinned", self._h)

    def run_device(self):
        _lib.call("mh_engine_run_device", self._h)

    def launch(self):
        _lib.call("mh_engine_launch", self._h)

    def stream(self) -> int:
        s = _vp()
        _lib.call("mh_engine_stream", self._h, ctypes.byref(s))
        return s.value or 0

    def input_ptr(self) -> int:
        p = _vp()
        _lib.call("mh_engine_input_ptr", self._h, ctypes.byref(p))
        return p.value

    def output_ptr(self) -> int:
        p = _vp()
        _lib.call("mh_engine_output_ptr", self._h, ctypes.byref(p))
        return p.value

    # -- introspection --------------------------------------------------------
    def _json(self, fn, size=1 << 16, *args):
        while True:
            buf = ctypes.create_string_buffer(size)
            try:
                _lib.call(fn, self._h, *args, buf, size)
                return json.loads(buf.value.decode())
            except _lib.HipError as e:
                if "buffer too small" not in str(e):
                    raise
                size *= 4

    def stats(self) -> dict:
        return self._json("mh_engine_stats")

    def plan(self) -> dict:
        return self._json("mh_engine_plan", 1 << 20)

    def op_times(self, reps: int = 20, only: str | None = None) -> list:
        """GPU time of every op of the compiled forward (or only the ops named
        ``only``) on its own: a list of {name, kind, us, flops, bytes}
        (mh_engine_op_times)."""
        return self._json("mh_engine_op_times", 1 << 20, reps, (only or "").encode())

    def forward_op_times(self, reps: int = 20) -> list:
        """GPU time of every op inside the forward: a list of {name, kind, us,
        flops, bytes}, us = difference of consecutive prefix-graph times, each
        over ``reps`` replays (mh_engine_forward_op_times)."""
        return self._json("mh_engine_forward_op_times", 1 << 20, reps)

    def close(self):
        if self._h is not None:
            _lib.call("mh_engine_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Decoder:
    """Greedy autoregressive decode with a KV cache over a compiled DecoderLM
    engine whose config has ``"attention": "textbook"`` (mh_decoder_*; no
    counterpart in the reference, whose attention has no per-position keys).

    ``prefill(ids [B, T0])`` runs the engine's forward and fills the caches;
    ``step(ids [B] or None)`` feeds one token per sequence; ``generate(n)``
    runs n greedy steps back to back on the device."""

    def __init__(self, engine: Engine, batch: int, max_len: int):
        self.engine = engine
        self.batch = int(batch)
        self.max_len = int(max_len)
        self.vocab = int(engine.config["vocab"])
        h = _vp()
        _lib.call("mh_decoder_create", ctypes.byref(h), engine._h, self.batch, self.max_len)
        self._h = h

    def _dt(self):
        return synth.storage_dtype(synth.DTYPE_CODES[self.engine.config.get("dtype", "float32")])

    def prefill(self, ids: np.ndarray, logits: bool = True):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        if ids.ndim != 2 or ids.shape[0] != self.batch:
            raise ValueError(f"prompt must be [batch={self.batch}, T0] int32")
        out = np.empty((self.batch, ids.shape[1], self.vocab), dtype=self._dt()) if logits else None
        _lib.call("mh_decoder_prefill", self._h, ids.ctypes.data_as(_vp), ids.shape[1],
                  out.ctypes.data_as(_vp) if out is not None else None)
        return out

    def step(self, ids=None):
        """-> (logits [B, V], next greedy ids [B])."""
        src = None
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(self.batch)
            src = ids.ctypes.data_as(_vp)
        logits = np.empty((self.batch, self.vocab), dtype=self._dt())
        nxt = np.empty(self.batch, dtype=np.int32)
        _lib.call("mh_decoder_step", self._h, src, logits.ctypes.data_as(_vp), nxt.ctypes.data_as(_vp))
        return logits, nxt

    def generate(self, n: int):
        """-> (tokens [n, B], device ms of the n steps)."""
        toks = np.empty((int(n), self.batch), dtype=np.int32)
        ms = ctypes.c_float()
        _lib.call("mh_decoder_generate", self._h, int(n), toks.ctypes.data_as(_vp), ctypes.byref(ms))
        return toks, float(ms.value)

    def position(self) -> int:
        p = ctypes.c_int()
        _lib.call("mh_decoder_position", self._h, ctypes.byref(p))
        return p.value

    def stats(self) -> dict:
        buf = ctypes.create_string_buffer(1 << 12)
        _lib.call("mh_decoder_stats", self._h, buf, len(buf))
        return json.loads(buf.value.decode())

    def close(self):
        if self._h is not None:
            _lib.call("mh_decoder_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
