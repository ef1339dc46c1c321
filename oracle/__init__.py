"""ORACLE — TEST INFRASTRUCTURE ONLY.

ctypes binding of ``liboracle_mul.so`` (the CPU restatement of the reference CPU backend's matmul,
``oracle/mul_oracle.cpp``) plus brute-force checkers.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the checker or the
reported CPU baseline; the product libraries never load it.

Pinning of each function (tests/test_oracle.py, tests/golden/):
  mul (int paths)      exact int64 brute force, low-byte closed forms, all-ones / identity KATs
  mul (fp32 paths)     exactly representable integer-valued fp32 sums; fp64 brute force (tolerance)
  widen (bf16/fp16)    RNE tables and numpy's IEEE fp16 conversion
  transpose_last2      numpy transpose
  result_type          the reference's compute_type table (include/core/type_traits.h:262-287)
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle_mul.so"

INT8, INT16, INT32, INT64, BFLOAT16, FLOAT16, FLOAT32, FLOAT64 = range(8)
NP = {INT8: np.int8, INT16: np.int16, INT32: np.int32, INT64: np.int64, BFLOAT16: np.uint16,
      FLOAT16: np.uint16, FLOAT32: np.float32, FLOAT64: np.float64}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "-B"], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.oracle_mul.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
        L.oracle_mul.restype = ctypes.c_int
        L.oracle_result_type.argtypes = [ctypes.c_int, ctypes.c_int]
        L.oracle_result_type.restype = ctypes.c_int
        L.oracle_compute_type.argtypes = [ctypes.c_int, ctypes.c_int]
        L.oracle_compute_type.restype = ctypes.c_int
        L.oracle_widen_f32.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_widen_f32.restype = None
        L.oracle_threads_used.argtypes = []
        L.oracle_threads_used.restype = ctypes.c_int
        L.oracle_transpose_last2.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                             ctypes.c_int64, ctypes.c_int64]
        L.oracle_transpose_last2.restype = None
        _lib = L
    return _lib


def result_type(dta: int, dtb: int) -> int:
    """Result dtype of the CPU backend's matmul (fp16/bf16 widened first)."""
    return lib().oracle_result_type(dta, dtb)


def compute_type(dta: int, dtb: int) -> int:
    return lib().oracle_compute_type(dta, dtb)


def mul(a: np.ndarray, dta: int, b: np.ndarray, dtb: int, variant: int = 0) -> np.ndarray:
    """``MulImpl<CPU>::execute`` on dense [b?, M, K] @ [b?, K, N] storage arrays.

    bf16/fp16 operands are passed as uint16 bit patterns.  variant: 0 reference choice,
    1 force ``mul_kernel_basic``, 2 force ``mul_kernel_tiled``.
    """
    a = np.ascontiguousarray(a, dtype=NP[dta])
    b = np.ascontiguousarray(b, dtype=NP[dtb])
    if a.ndim == 2:
        batch, (M, K), N = 1, a.shape, b.shape[-1]
        out_shape = (M, N)
    else:
        (batch, M, K), N = a.shape, b.shape[-1]
        out_shape = (batch, M, N)
    assert b.shape[-2] == K and (b.ndim == a.ndim)
    rt = result_type(dta, dtb)
    c = np.zeros(out_shape, dtype=NP[rt])
    got = lib().oracle_mul(dta, a.ctypes.data, dtb, b.ctypes.data, c.ctypes.data, batch, M, K, N, variant)
    assert got == rt, (got, rt)
    return c


def widen_f32(bits: np.ndarray, dt: int) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().oracle_widen_f32(dt, bits.ctypes.data, out.ctypes.data, bits.size)
    return out


def transpose_last2(x: np.ndarray) -> np.ndarray:
    """``ops::Transpose(x, {0, 2, 1})`` (or ``{1, 0}`` for 2-D), materialised."""
    x = np.ascontiguousarray(x)
    squeeze = x.ndim == 2
    x3 = x[None] if squeeze else x
    bt, r, c = x3.shape
    out = np.empty((bt, c, r), dtype=x.dtype)
    lib().oracle_transpose_last2(x.itemsize, x3.ctypes.data, out.ctypes.data, bt, r, c)
    return out[0] if squeeze else out


def threads_used() -> int:
    return lib().oracle_threads_used()


# ---- brute-force checkers -------------------------------------------------------------------

def exact_int(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Exact integer matmul as int64.  When every partial sum is below 2^53 in magnitude the fp64
    BLAS product is exact and is used (fast); otherwise numpy's int64 matmul."""
    a64, b64 = a.astype(np.int64), b.astype(np.int64)
    k = a.shape[-1]
    amax = int(np.abs(a64).max(initial=0))
    bmax = int(np.abs(b64).max(initial=0))
    if amax * bmax * max(k, 1) < 2 ** 53:
        return np.matmul(a64.astype(np.float64), b64.astype(np.float64)).astype(np.int64)
    return np.matmul(a64, b64)


def low_byte(x: np.ndarray) -> np.ndarray:
    """Low byte of an exact integer sum, as int8 (two's complement)."""
    return (np.asarray(x, dtype=np.int64) & 0xFF).astype(np.uint8).view(np.int8)


def f64_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.matmul(a.astype(np.float64), b.astype(np.float64))


def abs_bound(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """sum_k |a_ik| |b_kj|: the scale the relative-error tolerances are measured against."""
    return np.matmul(np.abs(a.astype(np.float64)), np.abs(b.astype(np.float64)))
