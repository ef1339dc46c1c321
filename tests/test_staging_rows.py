"""Compile-time check of the staged stores' rows per pass (staged_rows in gemm_mfma_impl.h), for a
sweep of wave-tile heights WM, padded row pitches and staging areas, by compiling a translation unit
of static_asserts for gfx950 (syntax only, no GPU).  A pass stores whole 16-row fragment blocks, so
the row count must be a multiple of 16 that divides WM; it must fit the staging area whenever 16 rows
do; and no larger such count may fit.  Halving WM, as an earlier helper did, gives 24 rows for
WM = 48 with a 528-byte pitch: the stores then wrote rows that no pass had staged.
"""
import subprocess

from tensorvia_amd import build_ext as be

WMS = [16, 32, 48, 64, 80, 96, 112, 128, 160, 192, 256]
PITCHES = [48, 80, 144, 272, 528, 1040, 2064]
AREAS = [9216, 18432, 36864]


def test_staged_rows_whole_blocks(tmp_path):
    src = tmp_path / "staged_rows_check.hip"
    cases = "\n".join(f"static_assert(ok<{w}, {p}, {a}>(), \"WM {w} pitch {p} area {a}\");"
                      for w in WMS for p in PITCHES for a in AREAS)
    src.write_text(f"""#include "gemm_mfma_impl.h"
template <int WM, int PITCH, int BYTES> constexpr bool ok() {{
    constexpr int r = tvk::staged_rows<WM, PITCH, BYTES>();
    if (r < 16 || r % 16 != 0 || WM % r != 0) return false;
    for (int q = r + 16; q <= WM; q += 16)
        if (WM % q == 0 && q * PITCH <= BYTES) return false;
    return r * PITCH <= BYTES || 16 * PITCH > BYTES;
}}
// The 48-row wave tile with 128 fp32 columns: 48 rows do not fit, 32 do not divide 48.
static_assert(tvk::staged_rows<48, 528, 18432>() == 16);
{cases}
""")
    r = subprocess.run([be.HIPCC, f"--offload-arch={be.ARCH}", "-std=c++20", "-fsyntax-only", "-w",
                        f"-I{be.INCLUDE}", f"-I{be.CSRC}", str(src)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
