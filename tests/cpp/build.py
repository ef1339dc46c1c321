"""Build the C++ API test programs (tests/cpp/bin/) against tensorvia_amd/libtensorvia.so."""
from __future__ import annotations

import os
from pathlib import Path

from tensorvia_amd import build_ext as be
from tensorvia_amd.host import build_host as bh

HERE = Path(__file__).resolve().parent
BIN = HERE / "bin"
PROGRAMS = ["host_api_test", "mul_driver", "init_driver", "copy_driver", "large_driver", "threads_driver"]


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


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build of the C++ API's CPU path: the
# host sources of libtensorvia.so compiled into the test program itself, so every pointer
# computation on view offsets, the staging-copy threads and the validation code run
# instrumented.  CPU only: the kernel library and the HIP runtime are linked as they are.
# A ThreadSanitizer build of the same program checks the memcpy thread pool's hand-offs.
SANITIZE_FLAGS = {"asan": ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"], "tsan": ["-fsanitize=thread"]}
SANITIZED = {"host_api_test_asan": ("host_api_test", "asan"), "host_api_test_tsan": ("host_api_test", "tsan")}


def build_sanitized(verbose: bool = False) -> None:
    BIN.mkdir(exist_ok=True)
    for exe, (prog, kind) in SANITIZED.items():
        out = BIN / exe
        tmp = out.with_suffix(".tmp")
        srcs = [str(bh.HOST / s) for s in bh.SOURCES] + [str(HERE / (prog + ".cpp"))]
        flags = [f for f in bh.CXXFLAGS if f != "-O2"] + ["-O1", "-g", "-fno-omit-frame-pointer"] + SANITIZE_FLAGS[kind]
        be._run([bh.CXX, *flags, *srcs, "-o", str(tmp), f"-L{be.PKG}", "-ltv_hip", f"-L{bh.ROCM}/lib",
                 "-lamdhip64", "-pthread", f"-Wl,-rpath,{be.PKG}", "-Wl,-rpath,$ORIGIN/../../../tensorvia_amd",
                 f"-Wl,-rpath,{bh.ROCM}/lib"], verbose)
        os.replace(tmp, out)


def binary(prog: str) -> Path:
    p = BIN / prog
    if not p.exists():
        build_sanitized() if prog in SANITIZED else build()
    return p


if __name__ == "__main__":
    import sys
    build_sanitized(verbose=True) if "--sanitize" in sys.argv else build(verbose=True)
