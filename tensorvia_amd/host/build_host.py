"""Build libtensorvia.so: the C++ Tensorvia API (Tensor, ops::Mul, HIP backend) over libtv_hip.so.

Host-only C++20 compiled with ROCm's clang++; links libamdhip64 and the kernel library, with an
$ORIGIN rpath so the pair loads from the package directory.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

from .. import build_ext as be

HOST = Path(__file__).resolve().parent
SOURCES = ["factory.cpp", "tensor.cpp", "hip_backend.cpp", "ops.cpp"]
CXX = os.environ.get("TV_HOST_CXX", "/opt/rocm/llvm/bin/clang++")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

CXXFLAGS = ["-std=c++20", "-O2", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__",
            f"-I{be.INCLUDE}", f"-I{ROCM}/include"]


def build(verbose: bool = False) -> Path:
    be.BUILD.mkdir(exist_ok=True)
    objs, jobs = [], []
    for src in SOURCES:
        s = HOST / src
        o = be.BUILD / ("host_" + src + ".o")
        objs.append(o)
        jobs.append([CXX, *CXXFLAGS, "-c", str(s), "-o", str(o)])
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        list(ex.map(lambda c: be._run(c, verbose), jobs))
    tmp = be.HOST_LIB.with_suffix(".so.tmp")
    be._run([CXX, "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
             f"-L{be.PKG}", "-ltv_hip", f"-L{ROCM}/lib", "-lamdhip64", "-pthread",
             "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib"], verbose)
    os.replace(tmp, be.HOST_LIB)
    build_tools(verbose)
    return be.HOST_LIB


# Programs built on libtensorvia.so: ops_mul_time times ops::Mul end to end as the reference's
# tests/mul.cpp does (bench.py runs it).
TOOLS = ["ops_mul_time"]
BIN = be.PKG / "bin"


def build_tools(verbose: bool = False) -> None:
    BIN.mkdir(exist_ok=True)
    for prog in TOOLS:
        out = BIN / prog
        tmp = out.with_suffix(".tmp")
        be._run([CXX, *CXXFLAGS, "-Werror=format", str(HOST / (prog + ".cpp")), "-o", str(tmp), f"-L{be.PKG}", "-ltensorvia", "-ltv_hip",
                 f"-L{ROCM}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN/..", f"-Wl,-rpath,{ROCM}/lib"], verbose)
        os.replace(tmp, out)
