"""Portable seeded synthetic data in MuNet storage formats.

The reference fills tensors with a thread-count-dependent generator
(src/backend/cpu_backend.hpp:1021-1038), so inputs and weights here come from
a host-independent SplitMix64 stream per tensor:

* seed   = FNV-1a-64 of ``"<base_seed>:<scope>:<name>"``
* u64_i  = splitmix64(seed + (i + 1) * 0x9E3779B97F4A7C15)
* uniform = (u64 >> 11) * 2**-53 in [0, 1)
* normal  = Box-Muller in float64 over consecutive uniform pairs
* storage = float64 -> float32 -> dtype codec (fp16 round-half-away and bf16
  round-to-nearest-even, the reference's codecs, src/types.hpp:239-317).

Storage arrays are numpy ``float32`` (fp32), ``uint16`` bit patterns
(fp16 / bf16) and ``int32`` (indices).
"""
from __future__ import annotations

import numpy as np

F32, F16, BF16, I32 = 0, 1, 2, 3
DTYPE_CODES = {"float32": F32, "float16": F16, "bfloat16": BF16, "int32": I32}
DTYPE_NAMES = {v: k for k, v in DTYPE_CODES.items()}
BASE_SEED = 20261201

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for byte in text.encode():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def splitmix64(seed: int, n: int) -> np.ndarray:
    idx = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, n: int) -> np.ndarray:
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, n: int) -> np.ndarray:
    pairs = (n + 1) // 2
    u = uniform01(seed, 2 * pairs)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log1p(-u1))
    th = 2.0 * np.pi * u2
    out = np.empty(2 * pairs, dtype=np.float64)
    out[0::2] = r * np.cos(th)
    out[1::2] = r * np.sin(th)
    return out[:n]


def tensor_seed(scope: str, name: str, base_seed: int = BASE_SEED) -> int:
    return fnv1a64(f"{base_seed}:{scope}:{name}")


# ---- storage codecs -------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """bf16 round-to-nearest-even, no NaN special case (types.hpp:311-317)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))
    return ((b >> np.uint64(16)) & np.uint64(0xFFFF)).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """fp16 with round-half-away-from-zero on the magnitude (types.hpp:239-278)."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (bits >> 16) & 0x8000
    raw_exp = (bits >> 23) & 0xFF
    man = bits & 0x7FFFFF
    e = raw_exp - 127 + 15
    out = np.zeros(bits.shape, dtype=np.int64)
    nanf = raw_exp == 0xFF
    out = np.where(nanf, sign | np.where(man != 0, 0x7E00, 0x7C00), out)
    sub = (~nanf) & (e <= 0)
    tiny = sub & (e < -10)
    shift = np.clip(1 - e, 0, 31)
    sh = (man | 0x800000) >> shift
    out = np.where(sub & ~tiny, sign | ((sh + 0x1000) >> 13), out)
    out = np.where(tiny, sign, out)
    norm = (~nanf) & (e > 0)
    rm = (man + 0x1000) >> 13
    carry = rm == 0x400
    e2 = np.where(carry, e + 1, e)
    val = np.where(carry, sign | (e2 << 10), sign | (e << 10) | (rm & 0x3FF))
    val = np.where(e2 >= 31, sign | 0x7C00, val)
    out = np.where(norm, val, out)
    return out.astype(np.uint16)


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def encode(x: np.ndarray, dt: int) -> np.ndarray:
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32)
    if dt == F32:
        return x32
    if dt == F16:
        return f32_to_f16_bits(x32)
    if dt == BF16:
        return f32_to_bf16_bits(x32)
    raise ValueError(f"cannot encode floats as dtype {dt}")


def decode(x: np.ndarray, dt: int) -> np.ndarray:
    if dt == F32:
        return np.asarray(x, dtype=np.float32)
    if dt == F16:
        return f16_bits_to_f32(x)
    if dt == BF16:
        return bf16_bits_to_f32(x)
    if dt == I32:
        return np.asarray(x).astype(np.float32)
    raise ValueError(dt)


def storage_dtype(dt: int):
    return {F32: np.float32, F16: np.uint16, BF16: np.uint16, I32: np.int32}[dt]


def elem_size(dt: int) -> int:
    return 2 if dt in (F16, BF16) else 4


# ---- initialisers ---------------------------------

def make_tensor(scope: str, name: str, shape, dt: int, kind: str, **kw) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    seed = tensor_seed(scope, name, kw.get("base_seed", BASE_SEED))
    if kind == "zeros":
        vals = np.zeros(n)
    elif kind == "ones":
        vals = np.ones(n)
    elif kind == "uniform":
        lo, hi = kw.get("low", 0.0), kw.get("high", 1.0)
        vals = lo + (hi - lo) * uniform01(seed, n)
    elif kind == "normal":
        vals = kw.get("mean", 0.0) + kw.get("std", 1.0) * normal(seed, n)
    elif kind == "randint":
        hi = kw["high"]
        ids = (splitmix64(seed, n) % np.uint64(hi)).astype(np.int32)
        return ids.reshape(shape)
    else:
        raise ValueError(kind)
    return encode(vals, dt).reshape(shape)
