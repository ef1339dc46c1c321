"""Build the C++ API test programs (tests/cpp/bin/) against tensorvia_amd/libtensorvia.so."""
from __future__ import annotations

import os
from pathlib import Path

from tensorvia_amd import build_ext as be
from tensorvia_amd.host import build_host as bh

HERE = Path(__file__).resolve().parent
BIN = HERE / "bin"
PROGRAMS = ["host_api_test", "mul_driver", "init_driver", "copy_driver"]


def build(verbose: bool = False) -> None:
    BIN.mkdir(exist_ok=True)
    for prog in PROGRAMS:
        out = BIN / prog
        tmp = out.with_suffix(".tmp")
        be._run([bh.CXX, *bh.CXXFLAGS, str(HERE / (prog + ".cpp")), "-o", str(tmp),
                 f"-L{be.PKG}", "-ltensorvia", "-ltv_hip", f"-L{bh.ROCM}/lib", "-lamdhip64",
                 f"-Wl,-rpath,{be.PKG}", "-Wl,-rpath,$ORIGIN/../../../tensorvia_amd",
                 f"-Wl,-rpath,{bh.ROCM}/lib"], verbose)
        os.replace(tmp, out)


def binary(prog: str) -> Path:
    p = BIN / prog
    if not p.exists():
        build()
    return p
