"""The packed kernels as programs, and the plugin-buffer path's host logic (CPU, no GPU).

The reference's ``_matrix_program`` gives every LinAlg kernel slots (out, a, b) and
``Estimates(flops = 2 m n k, bytes = m n out + m k a + k n b)`` (codegen/linalg.py:37-58).
Here the estimates count packed operands at their packed size plus scales, and must equal the
algorithmic byte and flop counts of the measured configurations.
"""

import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest

from tinygrad_mi355x.codegen import program as P

ROOT = Path(__file__).resolve().parent.parent


def test_plugin_path_imports_no_torch():
    """The runtime, renderer, the plugin-buffer packed path and the UOp layer (IR, linearizer,
    matmul rewrite, schedule runner) import no torch."""
    code = ("import sys; sys.path.insert(0, 'tinygrad-dx12_amd');"
            "import tinygrad_mi355x.codegen.program, tinygrad_mi355x.runtime.ops_mi355x,"
            " tinygrad_mi355x.runtime.graph, tinygrad_mi355x.compat, tinygrad_mi355x.uop.linearize,"
            " tinygrad_mi355x.codegen.uop_matmul, tinygrad_mi355x.runtime.schedule;"
            "assert 'torch' not in sys.modules, sorted(m for m in sys.modules if 'torch' in m)[:5]")
    subprocess.run([sys.executable, "-c", code], check=True, cwd=ROOT)


def fp4_desc(n, k, scaled=True):
    return P.PackedDesc("fp4_e2m1", (n, k), n * k // 2, 64 if scaled else None, "float8_e8m0fnu" if scaled else None,
                        32)


@pytest.mark.parametrize("m,mem", [(1, 31_232_000), (4, 31_342_592), (16, 31_784_960)])
def test_estimates_of_the_fp4_decode_gemv(m, mem):
    """FP4 E2M1 + E8M0/32 W [14336, 4096] x bf16 X [M, 4096] -> bf16: codes + scales + X + Y."""
    prog = P.weight_program(fp4_desc(14336, 4096), m, "bfloat16", 4096, "bfloat16", 14336)
    assert prog.name == "tgm_gemv" and prog.slots == ("out", "a", "b")
    assert prog.estimates == P.Estimates(2 * m * 14336 * 4096, mem)
    assert prog.local_size == (256, 1, 1) and prog.global_size[0] > 0


def test_estimates_of_the_measured_gemms():
    int4 = P.PackedDesc("int4", (4096, 4096), 4096 * 2048, 64, "float16", 32)
    assert P.weight_program(int4, 1, "float16", 4096, "float16", 4096).estimates.mem == 9_453_568
    fp6 = P.PackedDesc("fp6_e3m2", (11008, 4096), 11008 * 3072, 64, "float8_e8m0fnu", 32)
    prog = P.weight_program(fp6, 2048, "bfloat16", 4096, "bfloat16", 11008)
    assert prog.name == "tgm_gemm_w"
    assert prog.estimates == P.Estimates(184_683_593_728, 97_091_584)
    square = P.mx_program(fp4_desc(8192, 8192), fp4_desc(8192, 8192), "bfloat16", 8192)
    assert square.estimates == P.Estimates(1_099_511_627_776, 205_520_896)
    wide = P.mx_program(fp4_desc(4096, 4096), fp4_desc(14336, 4096), "bfloat16", 14336)
    assert wide.estimates == P.Estimates(481_036_337_152, 157_548_544)
    dense = P.dense_program("bfloat16", 128, 64, "bfloat16", 256, 64, 64, "float32", 256)
    assert dense.estimates == P.Estimates(2 * 128 * 256 * 64, 128 * 64 * 2 + 256 * 64 * 2 + 128 * 256 * 4)
    assert P.dense_program("float8_e4m3fn", 8, 128, "float8_e5m2", 8, 128, 128, "float32", 8).name == "tgm_gemm_fp8"
    with pytest.raises(ValueError):  # per-tensor scales belong to FP8 operands only
        P.dense_program("bfloat16", 8, 64, "bfloat16", 8, 64, 64, "float32", 8, scale_a=4096)


def test_program_arguments_follow_the_c_abi():
    """The program's argument tuples have the arity of the C entry points (checked against the
    ctypes signatures) and put the slots where the headers say."""
    from tinygrad_mi355x.runtime import library as L

    progs = [P.unpack_program(fp4_desc(64, 64), "float32"),
             P.weight_program(fp4_desc(64, 128), 4, "bfloat16", 128, "float32", 64),
             P.weight_program(fp4_desc(64, 128), 64, "bfloat16", 128, "float32", 64),
             P.mx_program(fp4_desc(64, 128), fp4_desc(32, 128, False), "float32", 32),
             P.dense_program("float16", 8, 64, "float16", 8, 64, 64, "float32", 8)]
    for prog in progs:
        args = prog._args(111, 222, 333, 444)
        assert len(args) == len(L.SIGNATURES[prog.name]), prog.name
        assert args[-1] == 444 and 111 in args and 222 in args
    # tgm_gemm_w takes the activations first, the packed weight fifth
    gw = progs[2]._args(111, 222, 333, 444)
    assert gw[0] == 333 and gw[4] == 222 and gw[11] == 111


class FakeBuffer(SimpleNamespace):
    pass


def test_packed_buffer_validation_mirrors_packed_tensor():
    """dx12.py:32-47: the same ValueError messages over plugin buffers."""
    dev = object()
    buf = FakeBuffer(dev=dev, address=4096, size=8)
    with pytest.raises(ValueError, match="unknown packed format"):
        P.PackedBuffer(buf, "int3", (1,))
    with pytest.raises(ValueError, match="nonnegative dimensions"):
        P.PackedBuffer(buf, "int4", ())
    with pytest.raises(ValueError, match="device buffer"):
        P.PackedBuffer(b"\0" * 8, "int4", (2,))
    with pytest.raises(ValueError, match="smaller than the declared shape"):
        P.PackedBuffer(buf, "fp6_e3m2", (11,))
    with pytest.raises(ValueError, match="block size must be positive"):
        P.PackedBuffer(buf, "int4", (2,), block_size=0)
    scales = P.Matrix(FakeBuffer(dev=dev, address=0, size=4), "float16", (1, 2))
    with pytest.raises(ValueError, match="incompatible shape or device"):
        P.PackedBuffer(buf, "int4", (1, 8), scales, 2)
    other = P.Matrix(FakeBuffer(dev=object(), address=0, size=8), "float16", (1, 4))
    with pytest.raises(ValueError, match="incompatible shape or device"):
        P.PackedBuffer(buf, "int4", (1, 8), other, 2)
    ok = P.PackedBuffer(buf, "fp4_e2m1", (2, 8), P.Matrix(FakeBuffer(dev=dev, address=0, size=8), "float8_e8m0fnu",
                                                           (2, 1)))
    assert ok.default_dtype() == "float32" and ok.desc().scale_bytes == 2
    assert P.PackedBuffer(buf, "int4", (4,)).default_dtype() == "int32"


def test_zero_work_programs_return_without_a_launch():
    """Zero work: ``0.0 if wait else None`` without touching the device (the reference's Program)."""
    prog = P.unpack_program(P.PackedDesc("int4", (0, 32), 0), "float32")
    buf = FakeBuffer(dev=object(), address=0, size=0)
    assert prog(buf, buf, wait=True) == 0.0 and prog(buf, buf) is None


def test_plugin_path_argument_errors():
    dev = object()
    x = P.Matrix(FakeBuffer(dev=dev, address=0, size=256), "bfloat16", (2, 64))
    w = P.PackedBuffer(FakeBuffer(dev=dev, address=0, size=64), "fp4_e2m1", (2, 32))
    with pytest.raises(ValueError, match="compatible rank-two shapes"):
        P.matmul_nt(x, w)
    w2 = P.PackedBuffer(FakeBuffer(dev=object(), address=0, size=64), "fp4_e2m1", (2, 64))
    with pytest.raises(ValueError, match="one device"):
        P.matmul_nt(x, w2)
    w64 = P.PackedBuffer(FakeBuffer(dev=dev, address=0, size=64), "fp4_e2m1", (2, 64))
    with pytest.raises(ValueError, match="bf16, f16 or f32"):
        P.matmul_nt(x, w64, dtype="int8")
    with pytest.raises(ValueError, match="matching vector"):
        P.matvec(w, x)
