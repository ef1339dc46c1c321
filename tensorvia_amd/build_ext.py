"""Build the gfx950 HIP kernel library (libtv_hip.so) and the C++ Tensorvia host library.

Everything is compiled in-tree with hipcc so the shared objects travel with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
BUILD = PKG / "_build"
INCLUDE = ROOT / "include"

KERNEL_LIB = PKG / "libtv_hip.so"
HOST_LIB = PKG / "libtensorvia.so"

ARCH = os.environ.get("TV_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed fp32 ALU ops stay disabled (the compiler would otherwise form v_pk_*_f32 from float code).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

KERNEL_SOURCES = ["gemm_mfma_f32.hip", "gemm_mfma_bf16.hip", "gemm_mfma_f16.hip", "gemm_mfma_i8.hip",
                  "gemm_dispatch.hip", "gemv.hip", "gemm_simt.hip", "repack.hip", "elementwise.hip", "capi.hip"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l and "--hip-link" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _stale(target: Path, deps: list[Path]) -> bool:
    if not target.exists():
        return True
    t = target.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def build_kernels(verbose: bool = False, force: bool = True) -> Path:
    """Compile libtv_hip.so (the extern "C" kernel library) for ``ARCH``."""
    BUILD.mkdir(exist_ok=True)
    headers = [INCLUDE / "tensorvia_hip.h", CSRC / "tv_kernels.h", CSRC / "gemm_mfma_impl.h", CSRC / "gemm_dma_impl.h"]
    jobs = []
    objs = []
    for src in KERNEL_SOURCES:
        s = CSRC / src
        o = BUILD / (src + ".o")
        objs.append(o)
        if force or _stale(o, [s] + headers):
            jobs.append([HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall",
                         "-Wno-unused-function", *DEVICE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}",
                         "-c", str(s), "-o", str(o)])
    with ThreadPoolExecutor(max_workers=min(8, max(1, len(jobs)))) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    tmp = KERNEL_LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, KERNEL_LIB)
    return KERNEL_LIB


# Measurement programs (tensorvia_amd/bin/): lds_bank_probe issues one LDS access pattern of the
# GEMM kernels per launch, for rocprofv3's LDS bank-conflict counter.
PROBES = ["lds_bank_probe"]


def build_probes(verbose: bool = False) -> None:
    out_dir = PKG / "bin"
    out_dir.mkdir(exist_ok=True)
    for prog in PROBES:
        out = out_dir / prog
        tmp = out.with_suffix(".tmp")
        _run([HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-Wall", *DEVICE_FLAGS,
              str(CSRC / (prog + ".hip")), "-o", str(tmp)], verbose)
        os.replace(tmp, out)


def build(verbose: bool = False) -> None:
    build_kernels(verbose=verbose)
    build_probes(verbose=verbose)
    host = PKG / "host"
    if (host / "build_host.py").exists():
        from .host import build_host  # noqa: WPS433
        build_host.build(verbose=verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
