"""Loader for the committed golden vectors (tests/golden/golden.npz)."""
from __future__ import annotations

from pathlib import Path

import numpy as np

PATH = Path(__file__).resolve().parent / "golden.npz"


def load() -> dict:
    z = np.load(PATH, allow_pickle=False)
    cases: dict = {}
    for key in z.files:
        name, field = key.split("__")
        cases.setdefault(name, {})[field] = z[key]
    return cases
