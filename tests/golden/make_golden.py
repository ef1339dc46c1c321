"""Writes tests/golden/golden.npz: small seeded matmul cases with brute-force expected outputs.

The reference holds no golden vectors for this path (its tests/mul.cpp only times), so the expected
outputs here come from brute force that does not share code with the oracle restatement:
exact int64 sums (int8: their low byte) and fp64 sums of integer-valued operands, which every fp32
accumulation order reproduces exactly; half-precision outputs are those exact sums rounded once
(round-to-nearest-even).  Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from tensorvia_amd import rng  # noqa: E402

OUT = Path(__file__).resolve().parent / "golden.npz"

INT8, INT16, INT32, INT64, BFLOAT16, FLOAT16, FLOAT32, FLOAT64 = range(8)


def ints(seed, shape, lo, hi, dt):
    return rng.uniform_int(seed, int(np.prod(shape)), lo, hi).astype(dt).reshape(shape)


def low_byte(x):
    return (x.astype(np.int64) & 0xFF).astype(np.uint8).view(np.int8)


def main() -> None:
    cases = {}

    def add(name, a, dta, b, dtb, c, dtc, b_layout="nk"):
        cases[name] = dict(a=a, b=b, c=c, meta=np.array([dta, dtb, dtc, {"nk": 0, "kn_t": 1}[b_layout]], np.int64))

    # int8: low byte of the exact sum (odd shapes, tails in every dim)
    a = ints(101, (37, 129), -128, 127, np.int8)
    b = ints(102, (129, 53), -128, 127, np.int8)
    add("int8_37x129x53", a, INT8, b, INT8, low_byte(a.astype(np.int64) @ b.astype(np.int64)), INT8)
    a = ints(103, (3, 20, 70), -10, 10, np.int8)
    b = ints(104, (3, 70, 33), -10, 10, np.int8)
    add("int8_batched_3x20x70x33", a, INT8, b, INT8, low_byte(np.matmul(a.astype(np.int64), b.astype(np.int64))), INT8)
    # int8 -> int32 full sum
    a = ints(105, (19, 300), -128, 127, np.int8)
    b = ints(106, (300, 24), -128, 127, np.int8)
    add("int8_i32out_19x300x24", a, INT8, b, INT8, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32), INT32)

    # fp32, integer-valued: exact
    a = ints(107, (45, 77), -8, 8, np.float32)
    b = ints(108, (77, 61), -8, 8, np.float32)
    add("fp32_45x77x61", a, FLOAT32, b, FLOAT32, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32), FLOAT32)

    # bf16 / fp16 integer-valued: exact fp32 sums, rounded once to the output type
    x = ints(109, (33, 40), -4, 4, np.float32)
    y = ints(110, (40, 72), -4, 4, np.float32)
    exact = (x.astype(np.float64) @ y.astype(np.float64)).astype(np.float32)
    add("bf16_33x40x72", rng.f32_to_bf16_bits(x), BFLOAT16, rng.f32_to_bf16_bits(y), BFLOAT16,
        rng.f32_to_bf16_bits(exact), BFLOAT16)
    add("bf16_f32out_33x40x72", rng.f32_to_bf16_bits(x), BFLOAT16, rng.f32_to_bf16_bits(y), BFLOAT16, exact, FLOAT32)
    x = ints(111, (2, 21, 64), -6, 6, np.float32)
    kk = ints(112, (2, 50, 64), -6, 6, np.float32)  # K tensor [b, n, k]; B = K.permute(0, 2, 1)
    exact = np.matmul(x.astype(np.float64), kk.transpose(0, 2, 1).astype(np.float64)).astype(np.float32)
    add("fp16_qkT_2x21x64x50", rng.f32_to_f16_bits(x), FLOAT16, rng.f32_to_f16_bits(kk), FLOAT16,
        rng.f32_to_f16_bits(exact), FLOAT16, b_layout="kn_t")

    # decode-shaped (GEMV) bf16: x[1|8, 256] @ W[256, 96]
    for m in (1, 8):
        x = ints(113 + m, (m, 256), -3, 3, np.float32)
        w = ints(120 + m, (256, 96), -3, 3, np.float32)
        exact = (x.astype(np.float64) @ w.astype(np.float64)).astype(np.float32)
        add(f"bf16_gemv_{m}x256x96", rng.f32_to_bf16_bits(x), BFLOAT16, rng.f32_to_bf16_bits(w), BFLOAT16,
            rng.f32_to_bf16_bits(exact), BFLOAT16)

    flat = {}
    for name, d in cases.items():
        for k, v in d.items():
            flat[f"{name}__{k}"] = v
    np.savez_compressed(OUT, **flat)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(cases)} cases)")


if __name__ == "__main__":
    main()
