"""Host logic of the drop-in surface (CPU only): dtype rules, validation, registration,
the no-CPU-fallback rule and the C-ABI library's exports."""

import ctypes
import json
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

import tinygrad_mi355x
from tinygrad_mi355x import compat
from tinygrad_mi355x import dtype as D
from tinygrad_mi355x.codegen import linalg
from tinygrad_mi355x.codegen.decomp.mi355x import FORMATS, FP8_CANDIDATES, PackedTensor, matrix_intermediate
from tinygrad_mi355x.renderer.linalg import _accumulator
from tinygrad_mi355x.runtime import kernels as K

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tgm_packed.h"


# ----------------------------------------------------------------------------- dtype lattice
@pytest.mark.parametrize("a,b,expected", [
    (torch.float32, torch.float16, torch.float32),
    (torch.float32, torch.float64, torch.float64),
    (torch.float16, torch.bfloat16, torch.float32),
    (torch.float32, torch.float8_e8m0fnu, torch.float32),
    (torch.float32, torch.int64, torch.float32),
    (torch.int8, torch.float16, torch.float16),
    (torch.int8, torch.int32, torch.int32),
    (torch.uint8, torch.uint64, torch.uint64),
    (torch.int8, torch.uint8, torch.int16),
    (torch.float8_e4m3fn, torch.float8_e4m3fn, torch.float8_e4m3fn),
])
def test_least_upper_dtype(a, b, expected):
    assert D.least_upper_dtype(a, b) is expected
    assert D.least_upper_dtype(b, a) is expected


@pytest.mark.parametrize("dt,expected", [
    (torch.int8, torch.int32), (torch.uint8, torch.uint32), (torch.bool, torch.int32), (torch.float16, torch.float32),
    (torch.bfloat16, torch.float32), (torch.float8_e4m3fn, torch.float32), (torch.float64, torch.float64),
    (torch.int64, torch.int64), (torch.uint64, torch.uint64), (torch.float32, torch.float32),
])
def test_accumulator_widths(dt, expected):
    """ARCHITECTURE.md:294-299; test_linalg.py:221-230 (int8->int32, uint8->uint32), :119-127 (fp16->fp32)."""
    assert _accumulator(dt, dt) is expected


# ----------------------------------------------------------------------------- PackedTensor
def u8(values):
    return torch.tensor(values, dtype=torch.uint8)


@pytest.mark.parametrize("kwargs,message", [
    (dict(data=u8([0]), format="int3", shape=(1,)), "unknown packed format"),
    (dict(data=u8([0]), format="int4", shape=()), "nonnegative dimensions"),
    (dict(data=u8([0]), format="int4", shape=(-1,)), "nonnegative dimensions"),
    (dict(data=torch.zeros(2, dtype=torch.int8), format="int4", shape=(2,)), "flat uint8"),
    (dict(data=torch.zeros((1, 2), dtype=torch.uint8), format="int4", shape=(2,)), "flat uint8"),
    (dict(data=u8([0]), format="int4", shape=(3,)), "smaller than the declared shape"),
    (dict(data=u8([0, 0]), format="fp6_e3m2", shape=(3,)), "smaller than the declared shape"),
    (dict(data=u8([0]), format="int4", shape=(2,), block_size=0), "block size must be positive"),
    (dict(data=u8([0, 0]), format="int4", shape=(1, 4), scales=torch.ones(1, 2), block_size=4), "incompatible shape"),
    (dict(data=u8([0, 0]), format="int4", shape=(1, 4), scales=torch.ones(1, 1, device="meta"), block_size=4),
     "incompatible shape or device"),
])
def test_packed_validation(kwargs, message):
    """dx12.py:32-47: the same exception type and message for each rejected record."""
    with pytest.raises(ValueError, match=message):
        PackedTensor(**kwargs)


def test_packed_accepts_exact_storage_and_scales():
    p = PackedTensor(u8([0, 0, 0]), "fp6_e2m3", (4,))
    assert p.shape == (4,) and p.bits == 6
    s = PackedTensor(u8([0] * 5), "fp4_e2m1", (2, 5), torch.ones(2, 3), block_size=2)
    assert s.default_dtype() is torch.float32
    assert PackedTensor(u8([0]), "int4", (2,)).default_dtype() is torch.int32
    assert PackedTensor(u8([0]), "fp4_e2m1", (1, 2), torch.ones(1, 2, dtype=torch.float64), 1).default_dtype() is torch.float64


def test_formats_and_fp8_candidates():
    assert FORMATS["fp6_e3m2"] == (6, 3, 2, 3) and FORMATS["fp4_e2m1"] == (4, 2, 1, 1)
    assert FP8_CANDIDATES["fp6_e2m3"] == (torch.float8_e4m3fn,)


def test_matrix_intermediate_preserves_activations():
    """test_packed.py:118-124."""
    weights = PackedTensor(u8([0]), "fp6_e2m3", (1, 1))
    assert matrix_intermediate(torch.tensor([[1.125]], dtype=torch.float32), weights, True) is torch.float32
    assert matrix_intermediate(weights, weights, True) is torch.float8_e4m3fn
    fp4 = PackedTensor(u8([0]), "fp4_e2m1", (1, 1))
    e3m2 = PackedTensor(u8([0]), "fp6_e3m2", (1, 1))
    assert matrix_intermediate(fp4, e3m2) is torch.float8_e4m3fn
    assert matrix_intermediate(fp4, torch.zeros(1, 1, dtype=torch.float8_e5m2)) is torch.float8_e5m2
    assert matrix_intermediate(weights, torch.zeros(1, 1, dtype=torch.float8_e5m2)) is torch.float16


def test_matrix_intermediate_promotion():
    scaled = PackedTensor(u8([0]), "fp4_e2m1", (1, 2), torch.ones(1, 1, dtype=torch.float16))
    assert matrix_intermediate(scaled, torch.zeros(2, 1, dtype=torch.bfloat16)) is torch.float32
    wide = PackedTensor(u8([0]), "fp4_e2m1", (1, 2), torch.ones(1, 2, dtype=torch.float64), 1)
    assert matrix_intermediate(wide, wide) is torch.float64
    e8 = PackedTensor(u8([0]), "fp4_e2m1", (1, 2), torch.ones(1, 1).to(torch.float8_e8m0fnu))
    assert matrix_intermediate(e8, e8) is torch.float32
    int4 = PackedTensor(u8([0]), "int4", (1, 2))
    assert matrix_intermediate(int4, torch.zeros(2, 1, dtype=torch.int32)) is torch.int32
    assert matrix_intermediate(PackedTensor(u8([0]), "uint4", (1, 2)), torch.zeros(2, 1, dtype=torch.uint64)) is torch.uint64
    assert matrix_intermediate(int4, torch.zeros(2, 1, dtype=torch.bfloat16)) is torch.bfloat16


# ----------------------------------------------------------------------------- linalg validation
def test_matmul_argument_errors():
    a = torch.zeros(2, 3)
    with pytest.raises(ValueError, match="unknown matrix scope"):
        linalg.matmul(a, torch.zeros(3, 2), scope="Warp")
    with pytest.raises(ValueError, match="compatible rank-two"):
        linalg.matmul(a, torch.zeros(2, 3))
    with pytest.raises(ValueError, match="compatible rank-two"):
        linalg.matmul(torch.zeros(3), torch.zeros(3, 2))
    with pytest.raises(ValueError, match="one device"):
        linalg.matmul(a, torch.zeros(3, 2, device="meta"))
    with pytest.raises(ValueError, match="tile dimensions"):
        linalg.matmul(a, torch.zeros(3, 2), tile=(16, 0, 16))
    with pytest.raises(ValueError, match="matvec expects"):
        linalg.matvec(a, torch.zeros(2))
    with pytest.raises(ValueError, match="compatible rank-two"):
        linalg.matmul_nt(a, torch.zeros(3, 2))


def test_empty_operands_need_no_kernel():
    out = linalg.matmul(torch.zeros(2, 0), torch.zeros(0, 3))
    assert out.shape == (2, 3) and out.dtype is torch.float32 and not out.any()
    assert linalg.matmul(torch.zeros(0, 4), torch.zeros(4, 3)).shape == (0, 3)


def test_no_cpu_fallback():
    """CPU tensors never compute on the host: the product raises instead."""
    with pytest.raises(RuntimeError, match="HIP device"):
        PackedTensor(u8([0x21, 0x43]), "uint4", (2, 2)).unpack()
    with pytest.raises(RuntimeError, match="HIP device"):
        linalg.matmul(torch.ones(2, 2), torch.ones(2, 2))
    with pytest.raises(RuntimeError, match="HIP device"):
        linalg.matmul(PackedTensor(u8([0x21, 0x43]), "uint4", (2, 2)), torch.ones(2, 1))


# ----------------------------------------------------------------------------- registration
def test_register_is_idempotent_and_opens_no_hardware():
    assert compat.registered() and compat.DEVICES[0] == "MI355X"
    before = list(compat.DEVICES)
    tinygrad_mi355x.register()
    tinygrad_mi355x.register()
    assert compat.DEVICES == before
    code = ("import sys; sys.path.insert(0, %r); import torch, tinygrad_mi355x; "
            "assert not torch.cuda.is_initialized(); print('ok')" % str(ROOT / "tinygrad-dx12_amd"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.stdout.strip() == "ok", out.stderr


# ----------------------------------------------------------------------------- C ABI
def declared_functions() -> list[str]:
    text = "\n".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    return sorted(set(re.findall(r"^(?:int|int64_t|const char\*)\s+(tgm_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = K.load_library()
    names = declared_functions()
    assert {"tgm_unpack", "tgm_gemv", "tgm_gemm_w", "tgm_gemm_mx", "tgm_gemm_plain", "tgm_dec_attention"} <= set(names)
    for name in names:
        assert hasattr(lib, name), name
    assert set(K.EXPORTS) == set(names)
    assert lib.tgm_abi_version() == K.ABI_VERSION


def declared_arities() -> dict[str, int]:
    """Parameter count of every function declared in include/*.h."""
    text = "\n".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    found = {}
    for m in re.finditer(r"^(?:int|int64_t|const char\*)\s+(tgm_\w+)\(([^)]*)\);", text, flags=re.M):
        params = m.group(2).strip()
        found[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return found


def test_binding_arities_match_the_headers():
    """The ctypes argument lists have one entry per declared parameter, and every
    ``K.call("tgm_...", ...)`` in the package, the tests and the bench passes that many."""
    import ast

    arity = declared_arities()
    assert set(arity) == set(declared_functions())
    lib = K.load_library()
    for name, n in arity.items():
        argtypes = getattr(lib, name).argtypes
        assert argtypes is not None and len(argtypes) == n, name
    sources = [*(ROOT / "tinygrad-dx12_amd").rglob("*.py"), *(ROOT / "tests").glob("*.py"), ROOT / "bench.py",
               ROOT / "__graft_entry__.py"]
    calls = 0
    for path in sources:
        for node in ast.walk(ast.parse(path.read_text())):
            if (isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute) and node.func.attr == "call"
                    and node.args and isinstance(node.args[0], ast.Constant) and isinstance(node.args[0].value, str)
                    and node.args[0].value.startswith("tgm_")
                    and not any(isinstance(a, ast.Starred) for a in node.args)):
                name = node.args[0].value
                assert len(node.args) - 1 == arity[name], f"{path.name}:{node.lineno} {name}"
                calls += 1
    assert calls > 40


def test_invalid_arguments_are_rejected_without_a_gpu():
    """Argument validation runs on the host and maps to ValueError (no kernel is launched)."""
    with pytest.raises(ValueError, match="unknown packed format"):
        K.call("tgm_unpack", None, 0, 9, 1, 1, None, -1, 32, None, 13, None)
    with pytest.raises(ValueError, match="smaller than the declared shape"):
        K.call("tgm_unpack", None, 1, 0, 3, 3, None, -1, 32, None, 13, None)
    with pytest.raises(ValueError, match="M must be <= 16"):
        K.call("tgm_gemv", None, 2, 16, 128, None, -1, 32, None, 12, 17, 128, None, 12, 16, None)
    with pytest.raises(ValueError, match="FP4/FP6 format"):
        K.call("tgm_quantize_mx", None, 13, 1, 32, 0, 32, None, None, None)
    with pytest.raises(ValueError, match="4 or 6 bits"):
        K.call("tgm_pack_codes", None, 4, 5, None, None)
    assert K.load_library().tgm_last_error().decode().startswith("pack width")


def test_scaled_mfma_routes_reject_unsupported_pairs_without_a_gpu():
    """tgm_gemm_mx rejects integer codes and E3M2 x E3M2 (whose gfx950 MFMA sums are not exact);
    tgm_gemm_fp8 takes only FP8 dtypes.  All before any launch."""
    fmt = K.FORMAT_IDS
    with pytest.raises(K.UnsupportedKernel, match="not integers"):
        K.call("tgm_gemm_mx", 16, fmt["int4"], None, 64, 16, fmt["fp4_e2m1"], None, 64, 128, 16, 13, 64, None)
    with pytest.raises(K.UnsupportedKernel, match="E3M2 x E3M2"):
        K.call("tgm_gemm_mx", 16, fmt["fp6_e3m2"], None, 64, 16, fmt["fp6_e3m2"], None, 64, 128, 16, 13, 64, None)
    with pytest.raises(K.UnsupportedKernel, match="multiple of 128"):
        K.call("tgm_gemm_mx", 16, fmt["fp6_e2m3"], None, 64, 16, fmt["fp4_e2m1"], None, 64, 96, 16, 13, 64, None)
    with pytest.raises(ValueError, match="FP8 E4M3 / E5M2"):
        K.call("tgm_gemm_fp8", 16, 12, 128, 64, 16, 12, 128, 64, 128, None, None, 16, 13, 64, None)
    with pytest.raises(K.UnsupportedKernel, match="multiple of 128"):
        K.call("tgm_gemm_fp8", 16, 9, 96, 64, 16, 10, 96, 64, 96, None, None, 16, 13, 64, None)


def test_automatic_fallbacks_are_recorded_and_warned_once():
    """auto falls back to the exact-width GEMM (linalg.py:219-223) but does not hide it: every
    fallback is recorded with its reason, and one that drops a packed product or follows a
    native rejection warns once per operand key; explicit scopes still raise."""
    from tinygrad_mi355x.codegen import linalg
    from tinygrad_mi355x.renderer.linalg import GEMV

    linalg.fallbacks.clear()
    linalg.matrix_failures.clear()

    def rejected():
        raise K.UnsupportedKernel("tgm_gemv: no kernel for this shape")

    key = ("tgm_gemv", 1, "k1")
    with pytest.warns(linalg.MatrixFallbackWarning, match="no kernel for this shape"):
        assert linalg._dispatch(rejected, lambda: "plain", GEMV, "auto", key) == "plain"
    assert linalg.fallbacks[key] == "tgm_gemv: no kernel for this shape" and key in linalg.matrix_failures
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert linalg._dispatch(rejected, lambda: "plain", GEMV, "auto", key) == "plain"  # cached: no second warning
        # an ordinary product with no native kernel is recorded without a warning
        assert linalg._dispatch(None, lambda: "plain", None, "auto", (None, 2, "f32")) == "plain"
    assert (None, 2, "f32") in linalg.fallbacks
    with pytest.warns(linalg.MatrixFallbackWarning, match="no native kernel"):
        linalg._dispatch(None, lambda: "plain", None, "auto", (None, 3, "packed"), True)
    with pytest.raises(RuntimeError, match="candidate rejected"):
        linalg._dispatch(rejected, lambda: "plain", GEMV, "Wave", key)
    assert linalg._dispatch(None, lambda: "plain", None, "tiled", ("t",)) == "plain" and ("t",) not in linalg.fallbacks
    linalg.fallbacks.clear()
    linalg.matrix_failures.clear()


def test_matrix_routing_table():
    """Static kernel choice (the analogue of the reference's LinAlg capability query,
    linalg.py:90-133): every FP4 / FP6 pair, scaled (E8M0 / 32) or not, takes the scaled MFMA;
    integer codes and non-E8M0 scales do not; FP8 tensors take the FP8 GEMM."""
    from tinygrad_mi355x.codegen.linalg import _dense_kernel, choose_matrix
    from tinygrad_mi355x.codegen import program as P
    from tinygrad_mi355x.renderer.linalg import GEMM_DENSE, GEMM_FP8, GEMM_MX, GEMM_MX_GENERAL

    def packed(fmt, scales, k=64):
        n = 4
        data = u8([0] * (n * k * FORMATS[fmt][0] // 8))
        sc = None if scales is None else torch.ones(n, k // 32, dtype=scales)
        return PackedTensor(data, fmt, (n, k), sc, 32)

    f32 = torch.float32
    for fa in ("fp4_e2m1", "fp6_e2m3", "fp6_e3m2"):
        for fb in ("fp4_e2m1", "fp6_e2m3", "fp6_e3m2"):
            for sa in (None, torch.float8_e8m0fnu):
                for sb in (None, torch.float8_e8m0fnu):
                    for k in (128, 256):
                        a, b = packed(fa, sa, k), packed(fb, sb, k)
                        # only FP4 x FP4 with both scales and K % 256 == 0 runs the 256 x 256 kernel
                        fast = fa == fb == "fp4_e2m1" and sa is not None and sb is not None and k == 256
                        kernel = choose_matrix(b, a, matrix_intermediate(a, b), f32, 4)
                        assert kernel is (GEMM_MX if fast else GEMM_MX_GENERAL)
                        assert choose_matrix(b, a, matrix_intermediate(a, b), f32, 4, tile=kernel.tile) is kernel
                        prog = P.mx_program(a.desc(), b.desc(), "float32", 4)
                        assert prog.kernel is kernel and prog.global_size[0] == 1
    big = P.mx_program(P.PackedDesc("fp4_e2m1", (4096, 8192), 4096 * 4096, 1, "float8_e8m0fnu"),
                       P.PackedDesc("fp6_e2m3", (1024, 8192), 1024 * 6144, 1, "float8_e8m0fnu"), "bfloat16", 1024)
    assert big.kernel is GEMM_MX_GENERAL and big.global_size[0] == 16 * 8  # 256 x 128 tiles
    ints = packed("int4", None)
    assert choose_matrix(packed("fp4_e2m1", None), ints, matrix_intermediate(ints, ints), f32, 4) is None
    f16s = packed("fp4_e2m1", torch.float16)
    assert choose_matrix(f16s, packed("fp4_e2m1", None), f32, f32, 4) is None
    x8, y8 = torch.zeros(2, 128, dtype=torch.float8_e4m3fn), torch.zeros(2, 128, dtype=torch.float8_e5m2)
    assert _dense_kernel(x8, y8, f32, None, "auto") is GEMM_FP8
    assert _dense_kernel(x8, y8, f32, None, "tiled") is None
    assert _dense_kernel(torch.zeros(2, 2, dtype=torch.bfloat16), torch.zeros(2, 2, dtype=torch.bfloat16), f32, None,
                         "auto") is GEMM_DENSE
    assert _dense_kernel(x8, torch.zeros(2, 128, dtype=torch.bfloat16), f32, None, "auto") is None


def test_noalloc_split_k_rejects_oversized_partials_before_any_gpu_call():
    """The allocation-free split-K GEMM checks its partials against the static scratch size on the
    host: 4 splits of 4096 x 4096 fp32 partials (256 MiB) exceed the 32 MiB array."""
    lib = K.load_library()
    assert lib.tgm_gemm_w_split_noalloc_capacity() == 32 << 20
    with pytest.raises(ValueError, match="static scratch"):
        K.call("tgm_gemm_w_split_noalloc", None, 12, 4096, 4096, None, 2, 4096, 4096, None, 15, 32, None, 13, 4096, 4,
               None)


def test_noalloc_split_k_checks_the_stream_device_before_any_launch():
    """A product that fits the scratch, on a non-null stream: the entry point settles which device's
    scratch it may use (the stream's device must be the current one) before it launches anything.
    Without a usable GPU that check fails with TGM_E_INVALID instead of a launch."""
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the GPU tests cover the launch path")
    with pytest.raises(ValueError, match="current HIP device|hipStreamGetDevice"):
        K.call("tgm_gemm_w_split_noalloc", 16, 12, 64, 2048, 16, 2, 512, 2048, 16, 15, 32, 16, 13, 512, 4, 0x1000)


def test_header_enums_match_binding():
    text = HEADER.read_text()
    for name, value in K.FORMAT_IDS.items():
        enum = {"int4": "INT4", "uint4": "UINT4", "fp4_e2m1": "FP4_E2M1", "fp6_e2m3": "FP6_E2M3", "fp6_e3m2": "FP6_E3M2"}[name]
        assert re.search(rf"TGM_FMT_{enum} = {value},", text)
    assert "TGM_E8M0 = 15" in text and K.DTYPE_IDS[torch.float8_e8m0fnu] == 15
    assert "TGM_BF16 = 12" in text and K.DTYPE_IDS[torch.bfloat16] == 12


@pytest.mark.parametrize("fmt,sdt,bs,swiglu,fits", [
    ("fp4_e2m1", torch.float8_e8m0fnu, 32, True, True),
    ("fp4_e2m1", torch.float8_e8m0fnu, 32, False, True),
    ("fp4_e2m1", None, 32, False, True),
    ("fp4_e2m1", None, 32, True, False),
    ("fp4_e2m1", torch.float16, 32, False, False),
    ("int4", torch.float16, 128, False, True),
    ("uint4", torch.bfloat16, 64, False, True),
    ("int4", torch.float32, 32, False, True),
    ("int4", torch.float16, 256, False, False),
    ("int4", torch.float16, 128, True, False),
    ("fp6_e2m3", torch.float8_e8m0fnu, 32, False, False),
])
def test_decoder_fuses_norms_only_into_supported_weights(fmt, sdt, bs, swiglu, fits):
    """The one-token decoder folds RMSNorm into a projection only for weights that
    tgm_dec_norm_gemv takes; any other weight keeps the separate norm launch."""
    from tinygrad_mi355x.decoder import _norm_gemv_fits
    n, k = 64, 2048
    bits = FORMATS[fmt][0]
    data = torch.zeros(n * k * bits // 8, dtype=torch.uint8)
    scales = None
    if sdt is not None:
        scales = torch.full((n, k // bs), 127, dtype=torch.uint8).view(sdt) if sdt == torch.float8_e8m0fnu \
            else torch.ones((n, k // bs), dtype=sdt)
    assert _norm_gemv_fits(PackedTensor(data, fmt, (n, k), scales, bs), swiglu) is fits


def test_profile_commands_name_existing_bench_workloads():
    """Every rocprofv3 summary under profiles/ gives the command that made it; the workloads
    those commands select with --only must exist in bench.py."""
    root = Path(__file__).resolve().parents[1]
    sys.path.insert(0, str(root))
    try:
        import bench
    finally:
        sys.path.remove(str(root))
    keys = set(bench.EXTRAS) | {bench.PRIMARY}
    summaries = sorted((root / "profiles").glob("*.txt"))
    assert summaries
    for path in summaries:
        text = path.read_text()
        assert "rocprofv3" in text, path.name
        for key in re.findall(r"--only (\S+)", text):
            assert key in keys, (path.name, key)


def _write_csv(path: Path, rows: list[dict]) -> None:
    import csv

    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as fh:
        writer = csv.DictWriter(fh, fieldnames=list(rows[0]))
        writer.writeheader()
        writer.writerows(rows)


def test_profile_summary_from_rocprof_csvs(tmp_path):
    """bench.py --summarize-profile on synthetic rocprofv3 CSVs: the timed dispatches are the last
    ones of the matching kernel, counters are medians per dispatch scaled by the copy calibration,
    MfmaUtil is reported as rocprofv3 derives it, and the shader clock is GRBM_GUI_ACTIVE (summed
    over 8 XCCs) / 8 / the kernel's duration."""
    root = Path(__file__).resolve().parents[1]
    sys.path.insert(0, str(root))
    try:
        import bench
    finally:
        sys.path.remove(str(root))
    kernel = "void tgm::gemm_mx_fp4<4, 2>(unsigned char const*)"
    durations = [400_000] * 5 + [300_000, 290_000, 310_000]  # 5 warm-up dispatches, then 3 timed
    trace = [{"Kernel_Name": kernel, "Start_Timestamp": 1000 * i, "End_Timestamp": 1000 * i + d}
             for i, d in enumerate(durations)]
    trace.insert(2, {"Kernel_Name": "other_kernel", "Start_Timestamp": 0, "End_Timestamp": 5})
    _write_csv(tmp_path / "kt" / "run_kernel_trace.csv", trace)
    flops, nbytes = 2 * 8192 ** 3, 205_520_896
    run = {"workload": "fp4xfp4", "ms": 0.3, "flops": flops, "bytes": nbytes, "timed_dispatches": 3,
           "roofline": bench.mfma_roofline(flops, 0.3, bench.FP4_PEAK_TFLOPS, "dense MXFP4 MFMA")}
    (tmp_path / "kt" / "bench.json").write_text(json.dumps({"fp4_gemm_8192": run}))

    def counters(folder, name, values, kname=kernel):
        _write_csv(tmp_path / folder / "run_counter_collection.csv",
                   [{"Dispatch_Id": i, "Kernel_Name": kname, "Counter_Name": name, "Counter_Value": v}
                    for i, v in enumerate(values)])

    counters("fetch", "FETCH_SIZE", [100_000.0, 200_000.0, 150_000.0])
    counters("write", "WRITE_SIZE", [131_072.0] * 3)
    counters("cfetch", "FETCH_SIZE", [32_768.0], "__amd_rocclr_copyBuffer")
    counters("cwrite", "WRITE_SIZE", [65_536.0], "__amd_rocclr_copyBuffer")
    rows = []
    for i in range(2):
        rows += [{"Dispatch_Id": i, "Kernel_Name": kernel, "Counter_Name": "SQ_VALU_MFMA_BUSY_CYCLES",
                  "Counter_Value": 512_000.0},
                 {"Dispatch_Id": i, "Kernel_Name": kernel, "Counter_Name": "GRBM_GUI_ACTIVE", "Counter_Value": 4_800_000.0},
                 {"Dispatch_Id": i, "Kernel_Name": kernel, "Counter_Name": "MfmaUtil", "Counter_Value": 54.5}]
    _write_csv(tmp_path / "mfma" / "run_counter_collection.csv", rows)
    text = bench.summarize_profile(tmp_path, "fp4_gemm_8192")
    assert "timed: mean_ns=300000 median_ns=300000" in text
    # FETCH median 150000 KiB x 2 (copy: 32768 KiB read for 64 MiB) + WRITE 131072 KiB x 1
    assert f"traffic_bytes_per_launch={(150_000 * 2 + 131_072) * 1024}" in text
    assert "pmc MfmaUtil median 54.50 %" in text
    assert "GRBM_GUI_ACTIVE / 8 / timed median = 2.000 GHz" in text  # 4.8e6 / 8 cycles in 300 us
    assert f"algorithmic_flops_per_launch={flops}" in text
    assert "--only fp4_gemm_8192" in text and "--pmc MfmaUtil SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE" in text


def test_decoder_trace_summary(tmp_path):
    """bench.py --summarize-decoder: segments start at dec_embed; prefills are the segments with a
    prompt GEMM; decode summarises the graph replays after the eager first step, prefill the
    second of the last three prefills."""
    root = Path(__file__).resolve().parents[1]
    sys.path.insert(0, str(root))
    try:
        import bench
    finally:
        sys.path.remove(str(root))
    trace, t = [], 0

    def launch(name, us):
        nonlocal t
        trace.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
        t += int(us * 1000) + 500

    for p in range(5):  # 2 warm-up prefills, then the 3 timed ones
        launch("tgm::dec_embed", 1)
        launch("tgm::gemm_w_mx<2, true, true>", 100 + p)
        launch("tgm::dec_argmax", 2)
    launch("tgm::dec_embed", 1)  # the eager first decode step: excluded
    launch("tgm::gemv_rows_fp4<8>", 50)
    for s in range(3):  # graph replays
        launch("tgm::dec_embed", 1)
        launch("tgm::gemv_rows_fp4<8>", 10 + s)
        launch("tgm::dec_argmax", 2)
    _write_csv(tmp_path / "run_kernel_trace.csv", trace)
    (tmp_path / "bench.json").write_text(json.dumps({"decoder_b1": {"decode_ms_per_step": 0.4, "prefill_ms": 3.1}}))
    dec = bench.summarize_decoder(tmp_path, "decoder_b1", "decode")
    assert "summarised: 3 steps; kernels per step: 3.0; busy 14.0 us/step" in dec
    assert "     11.00    1.0    11.00  tgm::gemv_rows_fp4<8>" in dec
    pre = bench.summarize_decoder(tmp_path, "decoder_b1", "prefill")
    assert "summarised: 1 prefill; kernels per prefill: 3.0" in pre
    assert "    103.00    1.0   103.00  tgm::gemm_w_mx<2, true, true>" in pre
