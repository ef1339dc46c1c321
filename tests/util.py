"""Shared helpers for the parity tests: storage arrays <-> torch tensors, tolerances."""
from __future__ import annotations

import numpy as np

INT8, INT16, INT32, INT64, BFLOAT16, FLOAT16, FLOAT32, FLOAT64 = range(8)

_NP_STORAGE = {INT8: np.int8, INT16: np.int16, INT32: np.int32, INT64: np.int64, BFLOAT16: np.uint16,
               FLOAT16: np.uint16, FLOAT32: np.float32, FLOAT64: np.float64}


def to_torch(arr: np.ndarray, dt: int, device="cuda"):
    """Storage array (uint16 bits for half types) -> torch tensor of dtype ``dt`` on ``device``."""
    from tensorvia_amd.matmul import storage_to_torch
    return storage_to_torch(arr, dt, device)


def to_storage(t) -> np.ndarray:
    """torch tensor -> numpy storage array (uint16 bits for half types)."""
    from tensorvia_amd.matmul import torch_to_storage
    return torch_to_storage(t)


def to_f32(arr: np.ndarray, dt: int) -> np.ndarray:
    from tensorvia_amd import rng
    if dt == BFLOAT16:
        return rng.bf16_bits_to_f32(arr)
    if dt == FLOAT16:
        return rng.f16_bits_to_f32(arr)
    return np.asarray(arr, dtype=np.float64)


def assert_fp32_close(c: np.ndarray, ref: np.ndarray, bound: np.ndarray, K: int) -> None:
    """fp32 tolerance: |c - ref| <= 1e-5 * sqrt(K) * sum_k |a_ik| |b_kj|."""
    err = np.abs(c.astype(np.float64) - ref.astype(np.float64))
    tol = 1e-5 * np.sqrt(max(K, 1)) * bound
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} elements over tolerance; worst {np.max(err / np.maximum(tol, 1e-300)):.3g}x"


def assert_half_close(c: np.ndarray, ref: np.ndarray, bound: np.ndarray, K: int) -> None:
    """fp16/bf16 tolerance: |c - ref| <= 1e-2 * |ref| + 1e-5 * sqrt(K) * sum_k |a_ik| |b_kj|
    (1e-2 relative to the fp32-accumulated value, plus the fp32 accumulation-order allowance)."""
    err = np.abs(c.astype(np.float64) - ref.astype(np.float64))
    tol = 1e-2 * np.abs(ref.astype(np.float64)) + 1e-5 * np.sqrt(max(K, 1)) * bound
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} elements over tolerance; worst {np.max(err / np.maximum(tol, 1e-300)):.3g}x"
