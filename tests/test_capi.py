"""C-ABI checks that need no GPU: the library loads, exports every declared symbol, and rejects
bad descriptors with the documented codes before touching a device."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

import tensorvia_amd as tv
from tensorvia_amd import TvGemmArgs

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:int|void|const char\*)\s+(tv_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_the_exported_set():
    assert declared_functions() == set(tv.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(tv.KERNEL_LIB))
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_matches_header():
    text = (ROOT / "include" / "tensorvia_hip.h").read_text()
    v = int(re.search(r"#define TV_HIP_ABI_VERSION (\d+)", text).group(1))
    assert tv.lib().tv_hip_abi_version() == v
    ext = int(re.search(r"#define TV_MAX_EXTENT (\d+)", text).group(1))
    assert ext == tv.TV_MAX_EXTENT == 2**31 - 2**20 - 1


@pytest.mark.parametrize("struct,cname", [("TvGemmArgs", "tv_gemm_args"), ("TvRepackArgs", "tv_repack_args"),
                                         ("TvEpilogue", "tv_epilogue")])
def test_struct_layout_matches_c(tmp_path, struct, cname):
    S = getattr(tv, struct)
    fields = [f for f, _ in S._fields_]
    src = tmp_path / "off.c"
    src.write_text("#include <stdio.h>\n#include <stddef.h>\n#include \"tensorvia_hip.h\"\nint main(void){\n"
                   + "".join(f'printf("%zu\\n", offsetof({cname}, {f}));\n' for f in fields)
                   + f'printf("%zu\\n", sizeof({cname}));return 0;}}\n')
    exe = tmp_path / "off"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [getattr(S, f).offset for f in fields] + [ctypes.sizeof(S)]
    assert got == want


def _args(**kw):
    a = TvGemmArgs()
    a.dtype_a = a.dtype_b = a.dtype_c = tv.FLOAT32
    a.batch, a.M, a.N, a.K = 1, 4, 4, 4
    a.A, a.B, a.C = 16, 32, 48  # never dereferenced: every case below returns before a launch
    a.sa_m, a.sa_k, a.sb_k, a.sb_n, a.sc_b, a.sc_m, a.sc_n = 4, 1, 4, 1, 16, 4, 1
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _call(fn, a):
    return getattr(tv.lib(), fn)(ctypes.byref(a), None)


@pytest.mark.parametrize("fn", ["tv_hip_gemm", "tv_hip_gemv"])
def test_rejections(fn):
    assert getattr(tv.lib(), fn)(None, None) == tv.TV_E_NULL
    assert _call(fn, _args(dtype_a=9)) == tv.TV_E_DTYPE
    assert _call(fn, _args(dtype_c=-1)) == tv.TV_E_DTYPE
    assert _call(fn, _args(dtype_a=tv.INT8, dtype_b=tv.INT8, dtype_c=tv.FLOAT32)) == tv.TV_E_DTYPE
    assert _call(fn, _args(dtype_a=tv.BFLOAT16, dtype_b=tv.BFLOAT16, dtype_c=tv.FLOAT16)) == tv.TV_E_DTYPE
    assert _call(fn, _args(M=-1)) == tv.TV_E_SHAPE
    assert _call(fn, _args(K=1 << 40)) == tv.TV_E_SHAPE
    # Each size is accepted up to TV_MAX_EXTENT (2^31 - 2^20 - 1): one past it is rejected; at it the
    # call passes the size check and stops at the missing output pointer.
    for dim in ("batch", "M", "N", "K"):
        assert _call(fn, _args(**{dim: tv.TV_MAX_EXTENT + 1})) == tv.TV_E_SHAPE, dim
        assert _call(fn, _args(**{dim: tv.TV_MAX_EXTENT}, C=None)) == tv.TV_E_NULL, dim
    assert _call(fn, _args(C=None)) == tv.TV_E_NULL
    assert _call(fn, _args(A=None)) == tv.TV_E_NULL
    assert _call(fn, _args(flags=1)) == tv.TV_E_UNSUPPORTED
    # empty problems are valid no-ops
    assert _call(fn, _args(M=0, A=None, B=None, C=None)) == tv.TV_OK
    assert _call(fn, _args(batch=0)) == tv.TV_OK


@pytest.mark.parametrize("fn", ["tv_hip_gemm", "tv_hip_gemv", "tv_hip_gemm_noalloc"])
def test_stride_rejections(fn):
    """Negative strides along extents above 1, zero strides of C there, and operands spanning 2^56
    bytes or more are rejected before any launch; the same strides on an extent of 1 are ignored.
    Calls whose strides pass stop at the missing output pointer (checked after the strides)."""
    for f in ("sa_m", "sa_k", "sb_k", "sb_n", "sc_m", "sc_n"):
        assert _call(fn, _args(**{f: -4})) == tv.TV_E_SHAPE, f
    assert _call(fn, _args(batch=2, sa_b=-16)) == tv.TV_E_SHAPE
    assert _call(fn, _args(batch=2, sb_b=-16)) == tv.TV_E_SHAPE
    assert _call(fn, _args(batch=2, sc_b=-16, sa_b=16)) == tv.TV_E_SHAPE
    for f in ("sc_m", "sc_n"):
        assert _call(fn, _args(**{f: 0})) == tv.TV_E_SHAPE, f  # two outputs in one element
    assert _call(fn, _args(batch=2, sc_b=0)) == tv.TV_E_SHAPE
    # zero strides of A and B broadcast: accepted
    assert _call(fn, _args(batch=2, sa_b=0, sb_b=0, sa_m=0, sb_k=0, C=None)) == tv.TV_E_NULL
    # extent 1: the stride is ignored, whatever its value
    assert _call(fn, _args(M=1, sa_m=-(1 << 62), sc_m=0, C=None)) == tv.TV_E_NULL
    assert _call(fn, _args(sa_b=-(1 << 62), sb_b=1 << 62, sc_b=-5, C=None)) == tv.TV_E_NULL  # batch 1
    # K = 0 reads neither operand: their strides are not checked
    assert _call(fn, _args(K=0, sa_m=-4, sb_n=-1, C=None)) == tv.TV_E_NULL
    # span: (M - 1) * sa_m * 4 bytes against 2^56, also where the product overflows 64 bits
    assert _call(fn, _args(sa_m=(1 << 54) // 3 - 1, C=None)) == tv.TV_E_NULL
    assert _call(fn, _args(sa_m=(1 << 54) // 3 + 1)) == tv.TV_E_SHAPE
    assert _call(fn, _args(sc_n=1 << 61)) == tv.TV_E_SHAPE
    assert _call(fn, _args(batch=3, sb_b=(1 << 63) - 1)) == tv.TV_E_SHAPE


def test_repack_rejections():
    """tv_hip_repack rejects bad ranks, element sizes and shapes, and shapes whose element count
    overflows 64 bits, before any launch; a view with a zero extent is an empty no-op wherever the
    zero stands."""
    L = tv.lib()

    def call(shape, elem_size=2, src=64, dst=128):
        a = tv.TvRepackArgs()
        a.ndim, a.elem_size, a.src, a.dst = len(shape), elem_size, src, dst
        for i, n in enumerate(shape):
            a.shape[i], a.strides[i] = n, 1
        return L.tv_hip_repack(ctypes.byref(a), None)

    assert L.tv_hip_repack(None, None) == tv.TV_E_NULL
    assert call([2, 2], elem_size=3) == tv.TV_E_DTYPE
    assert call([2, -1]) == tv.TV_E_SHAPE
    assert call([1 << 40, 1 << 40]) == tv.TV_E_SHAPE  # 2^80 elements
    assert call([1 << 40, 1 << 40, 0], src=None, dst=None) == tv.TV_OK
    assert call([0, 1 << 40, 1 << 40], src=None, dst=None) == tv.TV_OK
    assert call([4, 4], src=None) == tv.TV_E_NULL
    a = tv.TvRepackArgs()
    a.ndim = tv.TV_MAX_DIMS + 1
    assert L.tv_hip_repack(ctypes.byref(a), None) == tv.TV_E_SHAPE


def test_elementwise_rejections():
    """Typecast / fill / random reject bad arguments before any launch, and n = 0 is a no-op."""
    L = tv.lib()
    p = ctypes.c_void_p(64)  # never dereferenced
    assert L.tv_hip_typecast(p, 9, p, tv.FLOAT32, 4, None) == tv.TV_E_DTYPE
    assert L.tv_hip_typecast(p, tv.INT8, p, -1, 4, None) == tv.TV_E_DTYPE
    assert L.tv_hip_typecast(p, tv.INT8, p, tv.BFLOAT16, 4, None) == tv.TV_E_DTYPE  # not in valid_casts
    assert L.tv_hip_typecast(p, tv.FLOAT64, p, tv.FLOAT16, 4, None) == tv.TV_E_DTYPE
    assert L.tv_hip_typecast(p, tv.INT8, p, tv.FLOAT32, -1, None) == tv.TV_E_SHAPE
    assert L.tv_hip_typecast(None, tv.INT8, p, tv.FLOAT32, 4, None) == tv.TV_E_NULL
    assert L.tv_hip_typecast(None, tv.INT8, None, tv.FLOAT32, 0, None) == tv.TV_OK
    assert L.tv_hip_fill(p, 8, 4, 1.0, None) == tv.TV_E_DTYPE
    assert L.tv_hip_fill(p, tv.INT8, -3, 1.0, None) == tv.TV_E_SHAPE
    assert L.tv_hip_fill(None, tv.INT8, 3, 1.0, None) == tv.TV_E_NULL
    assert L.tv_hip_fill(None, tv.INT8, 0, 1.0, None) == tv.TV_OK
    assert L.tv_hip_random(p, -2, 4, 0.0, 1.0, 1, None) == tv.TV_E_DTYPE
    assert L.tv_hip_random(p, tv.FLOAT32, 4, 2.0, 1.0, 1, None) == tv.TV_E_SHAPE  # min > max
    assert L.tv_hip_random(p, tv.FLOAT32, -1, 0.0, 1.0, 1, None) == tv.TV_E_SHAPE
    assert L.tv_hip_random(None, tv.FLOAT32, 4, 0.0, 1.0, 1, None) == tv.TV_E_NULL
    assert L.tv_hip_random(None, tv.FLOAT32, 0, 0.0, 1.0, 1, None) == tv.TV_OK
    L.tv_hip_inject_fault(tv.TV_E_INJECTED, 3)
    assert L.tv_hip_typecast(p, tv.INT8, p, tv.FLOAT32, 4, None) == tv.TV_E_INJECTED
    assert L.tv_hip_fill(p, tv.INT8, 4, 1.0, None) == tv.TV_E_INJECTED
    assert L.tv_hip_random(p, tv.INT8, 4, 0.0, 1.0, 1, None) == tv.TV_E_INJECTED
    L.tv_hip_inject_fault(0, 0)


def test_gemm_ex_rejections():
    """The fused epilogue serves float outputs of the matrix-core pairs only."""
    L = tv.lib()

    def call(args, **ep):
        e = tv.TvEpilogue()
        for k, v in ep.items():
            setattr(e, k, v)
        return L.tv_hip_gemm_ex(ctypes.byref(args), ctypes.byref(e), None)

    assert L.tv_hip_gemm_ex(None, None, None) == tv.TV_E_NULL
    assert call(_args(), act=5) == tv.TV_E_UNSUPPORTED
    assert call(_args(), act=-1) == tv.TV_E_UNSUPPORTED
    assert call(_args(), act=tv.ACT_RELU, reserved=1) == tv.TV_E_UNSUPPORTED
    assert call(_args(dtype_a=tv.INT8, dtype_b=tv.INT8, dtype_c=tv.INT8), act=tv.ACT_RELU) == tv.TV_E_UNSUPPORTED
    assert call(_args(dtype_a=tv.INT32, dtype_b=tv.INT32, dtype_c=tv.INT32), act=tv.ACT_RELU) == tv.TV_E_UNSUPPORTED
    assert call(_args(dtype_c=-1), act=tv.ACT_RELU) == tv.TV_E_DTYPE
    assert call(_args(M=0, A=None, B=None, C=None), act=tv.ACT_SILU) == tv.TV_OK
    # bias strides: negative ones are rejected, and the elements read must lie within 2^30 bytes
    # (one buffer resource), also where (M - 1) * stride overflows 64 bits
    assert call(_args(), act=tv.ACT_RELU, bias=64, sbias_m=-1) == tv.TV_E_SHAPE
    assert call(_args(), act=tv.ACT_RELU, bias=64, sbias_n=1 << 28) == tv.TV_E_UNSUPPORTED
    assert call(_args(), act=tv.ACT_RELU, bias=64, sbias_m=1 << 62) == tv.TV_E_UNSUPPORTED
    assert call(_args(batch=3), act=tv.ACT_RELU, bias=64, sbias_b=(1 << 63) - 1) == tv.TV_E_UNSUPPORTED
    L.tv_hip_inject_fault(tv.TV_E_INJECTED, 1)
    assert call(_args(), act=tv.ACT_RELU) == tv.TV_E_INJECTED
    L.tv_hip_inject_fault(0, 0)


def test_gemv_rejects_large_m_and_non_mfma_pairs():
    assert _call("tv_hip_gemv", _args(M=9)) == tv.TV_E_UNSUPPORTED
    assert _call("tv_hip_gemv", _args(dtype_a=tv.INT32, dtype_b=tv.INT32, dtype_c=tv.INT32)) == tv.TV_E_UNSUPPORTED


def test_mixed_pairs_must_use_cpu_result_type():
    # int8 x int16 -> int16 (compute_type); anything else is rejected
    assert _call("tv_hip_gemm", _args(dtype_a=tv.INT8, dtype_b=tv.INT16, dtype_c=tv.INT8)) == tv.TV_E_DTYPE
    # bf16 x fp16 -> fp32 (widened on the CPU backend), int64 x fp32 -> fp64
    assert _call("tv_hip_gemm", _args(dtype_a=tv.BFLOAT16, dtype_b=tv.FLOAT16, dtype_c=tv.BFLOAT16)) == tv.TV_E_DTYPE
    assert _call("tv_hip_gemm", _args(dtype_a=tv.INT64, dtype_b=tv.FLOAT32, dtype_c=tv.FLOAT32)) == tv.TV_E_DTYPE


def test_fault_injection_propagates_and_disarms():
    L = tv.lib()
    L.tv_hip_inject_fault(tv.TV_E_INJECTED, 2)
    a = _args(M=0)
    assert _call("tv_hip_gemm", a) == tv.TV_E_INJECTED
    assert _call("tv_hip_gemv", a) == tv.TV_E_INJECTED
    assert _call("tv_hip_gemm", a) == tv.TV_OK
    L.tv_hip_inject_fault(7, 1)  # a positive code reads as a hipError_t
    with pytest.raises(tv.TensorviaHipError) as e:
        tv.check(_call("tv_hip_gemm", a))
    assert e.value.code == 7
    L.tv_hip_inject_fault(0, 0)


def test_strerror_covers_codes():
    for code in (0, -1, -2, -3, -4, -5, -6):
        s = tv.strerror(code)
        assert s and "unknown" not in s
    assert "unknown" in tv.strerror(-99)
