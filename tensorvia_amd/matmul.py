"""Python mirror of ``ops::Mul`` over the C-ABI, for torch tensors that live on the GPU.

Validation follows the reference's ``ops::Mul`` (src/ops.cpp:540-556), extended as the HIP backend
is: a rank-3 A may multiply a rank-2 B, which is then broadcast over the batch (batch stride 0).
The result dtype follows the GPU backends' ``compute_type(a, b)`` (include/core/type_traits.h:270-287,
src/backend/cuda/mul.cu:63); ``out_dtype=FLOAT32`` for half inputs gives the CPU backend's widened
result type instead (src/backend/cpu/mul.cpp:110-112).
"""
from __future__ import annotations

import ctypes

import torch

from . import (BFLOAT16, FLOAT16, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, TvGemmArgs, check,
               lib)

_T2TV = {torch.int8: INT8, torch.int16: INT16, torch.int32: INT32, torch.int64: INT64,
         torch.bfloat16: BFLOAT16, torch.float16: FLOAT16, torch.float32: FLOAT32, torch.float64: FLOAT64}
_TV2T = {v: k for k, v in _T2TV.items()}


def torch_to_tv(dt: torch.dtype) -> int:
    try:
        return _T2TV[dt]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dt}") from None


def tv_to_torch(dt: int) -> torch.dtype:
    return _TV2T[dt]


def storage_to_torch(arr, dt: int, device="cuda") -> torch.Tensor:
    """Host storage array (uint16 bit patterns for bf16/fp16) -> torch tensor of tv dtype ``dt``."""
    import numpy as np
    arr = np.ascontiguousarray(arr)
    if dt in (BFLOAT16, FLOAT16):
        return torch.from_numpy(arr.view(np.int16)).view(tv_to_torch(dt)).to(device)
    return torch.from_numpy(arr).to(device)


def torch_to_storage(t: torch.Tensor):
    """torch tensor -> host numpy storage array (uint16 bit patterns for bf16/fp16)."""
    import numpy as np
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def compute_type(a: int, b: int) -> int:
    """Result dtype of a binary op (reference include/core/type_traits.h:270-287)."""
    if a == b:
        return a
    if a <= INT64 and b <= INT64:
        return max(a, b)
    if a > INT64 and b > INT64:
        return max(max(a, FLOAT32), max(b, FLOAT32))
    if a == INT64 or b == INT64:
        return FLOAT64
    return max(max(a, FLOAT32), max(b, FLOAT32))


def _check_shapes(a: torch.Tensor, b: torch.Tensor) -> None:
    """The reference's checks in its order (src/ops.cpp:542-556), with the broadcast extension."""
    if a.device != b.device:
        raise RuntimeError("Tensors a and b device mismatch!")
    if b.dim() != a.dim() and not (a.dim() == 3 and b.dim() == 2):
        raise RuntimeError(f"Tensors a and b must have the same rank,but got {a.dim()} and {b.dim()}")
    if a.dim() not in (2, 3):
        raise RuntimeError(f"Tensors a and b dims must be 2 or 3,but got {a.dim()}")
    if a.dim() == 3:
        if b.dim() == 3 and a.shape[0] != b.shape[0]:
            raise RuntimeError("Tensors a and b must have the same batch size")
        if a.shape[2] != b.shape[-2]:
            raise RuntimeError(f"Tensors common dim must match,but {a.shape[2]} and {b.shape[-2]}")
    elif a.shape[1] != b.shape[0]:
        # the reference's 2-d message names dimension 0 of both operands (src/ops.cpp:555)
        raise RuntimeError(f"Tensors common dim must match,but {a.shape[0]} and {b.shape[0]}")


def make_args(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor) -> TvGemmArgs:
    """Pack the strided descriptor: element strides, data pointers that include the view offset."""
    args = TvGemmArgs()
    args.dtype_a, args.dtype_b, args.dtype_c = torch_to_tv(a.dtype), torch_to_tv(b.dtype), torch_to_tv(c.dtype)
    args.flags = 0
    if a.dim() == 3:
        args.batch, args.M, args.K = a.shape
        args.sa_b, args.sa_m, args.sa_k = a.stride()
    else:
        args.batch = 1
        args.M, args.K = a.shape
        args.sa_b = 0
        args.sa_m, args.sa_k = a.stride()
    if b.dim() == 3:
        args.N = b.shape[2]
        args.sb_b, args.sb_k, args.sb_n = b.stride()
    else:
        args.N = b.shape[1]
        args.sb_b = 0
        args.sb_k, args.sb_n = b.stride()
    if c.dim() == 3:
        args.sc_b, args.sc_m, args.sc_n = c.stride()
    else:
        args.sc_b = 0
        args.sc_m, args.sc_n = c.stride()
    args.A, args.B, args.C = a.data_ptr(), b.data_ptr(), c.data_ptr()
    return args


def _out(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None, out_dtype: int | None) -> torch.Tensor:
    _check_shapes(a, b)
    dt = out_dtype if out_dtype is not None else compute_type(torch_to_tv(a.dtype), torch_to_tv(b.dtype))
    shape = (a.shape[0], a.shape[1], b.shape[-1]) if a.dim() == 3 else (a.shape[0], b.shape[-1])
    if out is None:
        out = torch.empty(shape, dtype=tv_to_torch(dt), device=a.device)
    elif tuple(out.shape) != shape or torch_to_tv(out.dtype) != dt:
        raise RuntimeError(f"out has shape {tuple(out.shape)}/{out.dtype}, expected {shape}/{tv_to_torch(dt)}")
    return out


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream if isinstance(stream, int) else stream.cuda_stream


def gemm(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None, out_dtype: int | None = None,
         stream=None) -> torch.Tensor:
    """C = A @ B on the HIP kernels (asynchronous on ``stream``, default torch's current stream)."""
    out = _out(a, b, out, out_dtype)
    args = make_args(a, b, out)
    check(lib().tv_hip_gemm(ctypes.byref(args), ctypes.c_void_p(_stream(stream))))
    return out


def gemv(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None, out_dtype: int | None = None,
         stream=None) -> torch.Tensor:
    """Skinny-M (M <= 8) path; raises TensorviaHipError(TV_E_UNSUPPORTED) if it does not serve the call."""
    out = _out(a, b, out, out_dtype)
    args = make_args(a, b, out)
    check(lib().tv_hip_gemv(ctypes.byref(args), ctypes.c_void_p(_stream(stream))))
    return out


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``ops::Mul`` / ``ops::matmul``: synchronous, like the reference (src/backend/cuda/mul.cu:122)."""
    c = gemm(a, b)
    torch.cuda.current_stream().synchronize()
    return c
