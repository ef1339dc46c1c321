"""Seeded, counter-based input generator and host-side dtype rounding (numpy).

The reference seeds one ``std::mt19937`` per OpenMP thread from the clock
(src/backend/cpu/initializer.cpp:18-36), so its ``Tensor::Random`` streams cannot be reproduced.
This generator keeps the reference's value distributions and is reproducible from a seed:

* element ``i`` of stream ``seed`` is the SplitMix64 output for counter ``i`` of a stream whose
  start is SplitMix64(seed) — any element can be generated independently (host or device);
* floats: ``lo + (hi - lo) * u`` in fp32 with ``u`` the top 24 bits / 2^24, then rounded to the
  target dtype with round-to-nearest-even (the reference's ``static_cast<T>(float)``,
  initializer.cpp:30-33);
* integers: inclusive ``[lo, hi]`` by multiply-shift of the top 32 bits
  (``uniform_int_distribution`` semantics, initializer.cpp:27-29);
* normals (the reference has none): Box-Muller over two 24-bit uniforms, computed in fp64 and
  rounded to fp32.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def raw_u64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs ``start .. start+n-1`` of the stream for ``seed``."""
    with np.errstate(over="ignore"):
        key = _mix(np.array([np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + GAMMA], dtype=np.uint64))[0]
        ctr = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        return _mix(key + ctr * GAMMA)


def uniform_f32(seed: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    u = (raw_u64(seed, n) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    return np.float32(lo) + np.float32(hi - lo) * u


def uniform_int(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    span = np.uint64(hi - lo + 1)
    top = raw_u64(seed, n) >> np.uint64(32)
    with np.errstate(over="ignore"):
        return (np.int64(lo) + ((top * span) >> np.uint64(32)).astype(np.int64))


def normal_f32(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    m = (n + 1) // 2
    v = raw_u64(seed, 2 * m)
    u1 = ((v[0::2] >> np.uint64(40)).astype(np.float64) + 1.0) * 2.0 ** -24
    u2 = (v[1::2] >> np.uint64(40)).astype(np.float64) * 2.0 ** -24
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mean + std * z[:n]).astype(np.float32)


# ---- dtype rounding (host) -------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round-to-nearest-even; NaN stays NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    with np.errstate(over="ignore"):
        r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bit patterns (numpy's conversion is round-to-nearest-even)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def make(kind: str, shape, seed: int, dtype: str, lo: float = -1.0, hi: float = 1.0,
         mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Seeded host tensor.  Returns storage arrays: uint16 bit patterns for bf16/fp16."""
    n = int(np.prod(shape))
    if dtype in ("int8", "int16", "int32", "int64"):
        v = uniform_int(seed, n, int(lo), int(hi)).astype(dtype)
        return v.reshape(shape)
    if kind == "uniform":
        f = uniform_f32(seed, n, lo, hi)
    elif kind == "normal":
        f = normal_f32(seed, n, mean, std)
    else:
        raise ValueError(kind)
    if dtype == "bfloat16":
        return f32_to_bf16_bits(f).reshape(shape)
    if dtype == "float16":
        return f32_to_f16_bits(f).reshape(shape)
    if dtype == "float32":
        return f.reshape(shape)
    if dtype == "float64":
        return f.astype(np.float64).reshape(shape)
    raise ValueError(dtype)
