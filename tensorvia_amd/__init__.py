"""tensorvia_amd — MI355X (gfx950) HIP backend for Tensorvia's ``ops::Mul`` (matmul) path.

The product is two in-tree shared objects:

* ``libtv_hip.so``     — hand-written gfx950 kernels behind the C-ABI in ``include/tensorvia_hip.h``;
* ``libtensorvia.so``  — the C++ Tensorvia API (``Tensor``, ``ops::Mul`` ...) with the HIP backend.

This module binds the C-ABI with ctypes for Python callers (tests and ``bench.py``); PyTorch only
supplies device memory and streams.  There is no CPU fallback: if the kernel library is missing,
``lib()`` raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

PKG = Path(__file__).resolve().parent
KERNEL_LIB = PKG / "libtv_hip.so"
HOST_LIB = PKG / "libtensorvia.so"

# via::DataType (reference include/core/type_traits.h:123-132)
INT8, INT16, INT32, INT64, BFLOAT16, FLOAT16, FLOAT32, FLOAT64 = range(8)
DTYPE_NAMES = {INT8: "int8", INT16: "int16", INT32: "int32", INT64: "int64",
               BFLOAT16: "bfloat16", FLOAT16: "float16", FLOAT32: "float32", FLOAT64: "float64"}

TV_OK = 0
TV_E_NULL, TV_E_SHAPE, TV_E_DTYPE, TV_E_UNSUPPORTED, TV_E_INJECTED, TV_E_NOMEM, TV_E_SCRATCH = -1, -2, -3, -4, -5, -6, -7

# Every symbol include/tensorvia_hip.h declares.
EXPORTED_SYMBOLS = ("tv_hip_gemm", "tv_hip_gemm_ex", "tv_hip_gemm_noalloc", "tv_hip_gemv", "tv_hip_repack", "tv_hip_typecast", "tv_hip_fill",
                    "tv_hip_random", "tv_hip_strerror", "tv_hip_abi_version", "tv_hip_inject_fault",
                    "tv_hip_inject_alloc_failure")


class TvGemmArgs(ctypes.Structure):
    """Mirror of ``tv_gemm_args`` (include/tensorvia_hip.h)."""

    _fields_ = [
        ("dtype_a", ctypes.c_int32), ("dtype_b", ctypes.c_int32), ("dtype_c", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("batch", ctypes.c_int64), ("M", ctypes.c_int64), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
        ("A", ctypes.c_void_p), ("sa_b", ctypes.c_int64), ("sa_m", ctypes.c_int64), ("sa_k", ctypes.c_int64),
        ("B", ctypes.c_void_p), ("sb_b", ctypes.c_int64), ("sb_k", ctypes.c_int64), ("sb_n", ctypes.c_int64),
        ("C", ctypes.c_void_p), ("sc_b", ctypes.c_int64), ("sc_m", ctypes.c_int64), ("sc_n", ctypes.c_int64),
    ]


# enum tv_act
ACT_NONE, ACT_RELU, ACT_SILU, ACT_SIGMOID, ACT_TANH = range(5)


class TvEpilogue(ctypes.Structure):
    """Mirror of ``tv_epilogue`` (include/tensorvia_hip.h)."""

    _fields_ = [("act", ctypes.c_int32), ("reserved", ctypes.c_int32), ("bias", ctypes.c_void_p),
                ("sbias_b", ctypes.c_int64), ("sbias_m", ctypes.c_int64), ("sbias_n", ctypes.c_int64)]


TV_MAX_DIMS = 8
TV_MAX_EXTENT = (1 << 31) - (1 << 20) - 1  # largest batch / M / N / K of the GEMM entry points


class TvRepackArgs(ctypes.Structure):
    """Mirror of ``tv_repack_args`` (include/tensorvia_hip.h)."""

    _fields_ = [("ndim", ctypes.c_int32), ("elem_size", ctypes.c_int32),
                ("shape", ctypes.c_int64 * TV_MAX_DIMS), ("strides", ctypes.c_int64 * TV_MAX_DIMS),
                ("src", ctypes.c_void_p), ("dst", ctypes.c_void_p)]


class TensorviaHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (code {code})")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Load libtv_hip.so (built by ``__graft_entry__.build()``); raise if it is not built."""
    global _lib
    if _lib is None:
        if not KERNEL_LIB.exists():
            raise RuntimeError(f"{KERNEL_LIB} is not built; run __graft_entry__.build() first")
        L = ctypes.CDLL(str(KERNEL_LIB))
        L.tv_hip_gemm.argtypes = [ctypes.POINTER(TvGemmArgs), ctypes.c_void_p]
        L.tv_hip_gemm.restype = ctypes.c_int
        L.tv_hip_gemm_ex.argtypes = [ctypes.POINTER(TvGemmArgs), ctypes.POINTER(TvEpilogue), ctypes.c_void_p]
        L.tv_hip_gemm_ex.restype = ctypes.c_int
        L.tv_hip_gemm_noalloc.argtypes = [ctypes.POINTER(TvGemmArgs), ctypes.c_void_p]
        L.tv_hip_gemm_noalloc.restype = ctypes.c_int
        L.tv_hip_gemv.argtypes = [ctypes.POINTER(TvGemmArgs), ctypes.c_void_p]
        L.tv_hip_gemv.restype = ctypes.c_int
        L.tv_hip_repack.argtypes = [ctypes.POINTER(TvRepackArgs), ctypes.c_void_p]
        L.tv_hip_repack.restype = ctypes.c_int
        L.tv_hip_typecast.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                                      ctypes.c_int64, ctypes.c_void_p]
        L.tv_hip_typecast.restype = ctypes.c_int
        L.tv_hip_fill.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p]
        L.tv_hip_fill.restype = ctypes.c_int
        L.tv_hip_random.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_float,
                                    ctypes.c_uint64, ctypes.c_void_p]
        L.tv_hip_random.restype = ctypes.c_int
        L.tv_hip_strerror.argtypes = [ctypes.c_int]
        L.tv_hip_strerror.restype = ctypes.c_char_p
        L.tv_hip_abi_version.argtypes = []
        L.tv_hip_abi_version.restype = ctypes.c_int
        L.tv_hip_inject_fault.argtypes = [ctypes.c_int, ctypes.c_int]
        L.tv_hip_inject_fault.restype = None
        L.tv_hip_inject_alloc_failure.argtypes = [ctypes.c_int]
        L.tv_hip_inject_alloc_failure.restype = None
        _lib = L
    return _lib


def strerror(code: int) -> str:
    return lib().tv_hip_strerror(code).decode()


def check(code: int) -> None:
    if code != TV_OK:
        raise TensorviaHipError(code, strerror(code))


from .matmul import gemm, gemv, make_args, matmul, torch_to_tv, tv_to_torch  # noqa: E402,F401
