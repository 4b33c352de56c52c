"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against the reference's own known-answer data
(tests/golden/reference_vectors.json, extracted from the reference's tests), against
an independent library (torch casts) or against brute force / closed forms, chosen so
that a dropped term, a wrong shift or a swapped operand fails.
"""

import ctypes
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import packed_oracle as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
ORACLE_LIB = Path(__file__).resolve().parent.parent / "oracle" / "liboracle_cpu.so"
FMT_IDS = {"int4": 0, "uint4": 1, "fp4_e2m1": 2, "fp6_e2m3": 3, "fp6_e3m2": 4}


# ----------------------------------------------------------------------------- decode goldens
@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
def test_complete_ocp_payloads(fmt):
    """Every payload including -0 (test_packed.py:87-101 with its GOLDEN table)."""
    positive = GOLDEN["golden_positive_values"]["values"][fmt]
    bits = O.bits_of(fmt)
    data = np.array(O.payload_bytes(list(range(1 << bits)), bits), np.uint8)
    actual = O.unpack(data, fmt, (1 << bits,))
    assert actual.dtype == np.float32
    assert actual.tolist() == [*positive, *[-x for x in positive]]
    assert math.copysign(1, actual[len(positive)]) == -1
    assert math.copysign(1, actual[0]) == 1


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
def test_integer_nibbles(fmt):
    data = np.array(O.payload_bytes(list(range(16)), 4), np.uint8)
    out = O.unpack(data, fmt, (16,))
    assert out.dtype == np.int32 and out.tolist() == GOLDEN["integer_nibbles"][fmt]


def test_unit_codes_decode_to_unit_values():
    """The harness's exact {-1, 0, 1} payloads (benchmark_dtypes.py:70-74)."""
    for fmt, table in GOLDEN["unit_codes"].items():
        if fmt == "source":
            continue
        for value, code in table.items():
            assert O.decode_values(np.array([code]), fmt)[0] == float(value)


def test_scales_stay_with_k_blocks():
    case = GOLDEN["scales_stay_with_k_blocks"]
    w = O.unpack(np.array(case["data"], np.uint8), case["format"], case["shape"],
                 np.array(case["scales"], np.int64), case["block_size"], scale_dtype="int64")
    assert w.dtype == np.float32
    assert (w.astype(np.float64) @ np.array(case["rhs"], np.float64)).tolist() == case["expected"]


def test_double_block_scales():
    case = GOLDEN["double_block_scales"]
    w = O.unpack(np.array(case["data"], np.uint8), case["format"], case["shape"],
                 np.array(case["scales"], np.float64), case["block_size"])
    assert w.dtype == np.float64 and w.tolist() == case["decoded"]
    assert (w @ np.array(case["rhs"])).tolist() == case["expected"]


def test_readme_uint4_example():
    case = GOLDEN["readme_uint4"]
    w = O.unpack(np.array(case["data"], np.uint8), "uint4", case["shape"])
    assert w.tolist() == case["unpacked"]
    assert (w @ np.array(case["column"])).tolist() == case["matmul"]


@pytest.mark.parametrize("case", GOLDEN["large_bit_positions"]["cases"])
def test_large_packed_bit_positions(case):
    """Word-group extraction equals the closed-form bit-stream formula near 2**31
    (test_packed.py:147-174): the oracle decodes a group-aligned window of the
    17-byte pattern storage and must match the reference test's own formula."""
    fmt, kind, scaled = case
    pattern = GOLDEN["large_bit_positions"]["pattern"]
    scale_cycle = GOLDEN["large_bit_positions"]["scales"]
    bits = O.bits_of(fmt)
    boundary = 2 ** 31 // bits if kind == "bit" else 2 ** 31
    group_bytes = bits // 2
    g0 = (boundary - 3) // 4
    window = np.array([pattern[(g0 * group_bytes + j) % 17] for j in range(8 * group_bytes)], np.uint8)
    raw = O.payloads(window, fmt, 32)
    for index in range(boundary - 3, boundary + 7):
        payload = int(raw[index - g0 * 4])
        expected_payload = O.payload_at(lambda j: pattern[j % 17], index, bits)
        assert payload == expected_payload
        value = O.decode_values(np.array([payload]), fmt)[0] if fmt != "uint4" else payload
        golden = GOLDEN["golden_positive_values"]["values"]
        expected = payload if fmt == "uint4" else golden[fmt][payload & 31] * (-1 if payload & 32 else 1)
        if scaled:
            expected *= scale_cycle[index // 32 % 3]
            value *= scale_cycle[index // 32 % 3]
        assert value == expected


# ----------------------------------------------------------------------------- FP8 / E8M0 / bf16
@pytest.mark.parametrize("fmt,target", [(f, t) for f, ts in O.FP8_CANDIDATES.items() for t in ts])
def test_fp8_direct_matches_library_cast(fmt, target):
    """dx12.py:78-92 re-encode == torch's fp32->fp8 cast of the exact decoded values."""
    p = np.arange(1 << O.bits_of(fmt), dtype=np.uint32)
    tt = {"fp8e4m3": torch.float8_e4m3fn, "fp8e5m2": torch.float8_e5m2}[target]
    ref = torch.from_numpy(O.decode_values(p, fmt)).to(tt).view(torch.uint8).numpy()
    assert np.array_equal(O.fp8_direct(p, fmt, target), ref)
    assert np.array_equal(O.unpack(O.pack_codes(p, O.bits_of(fmt)), fmt, (p.size,), dtype=target), ref)


def test_fp6_e2m3_has_no_e5m2_shortcut():
    """E2M3 values need 3 mantissa bits, so E5M2 is not an exact choice (dx12.py:11)."""
    assert O.FP8_CANDIDATES["fp6_e2m3"] == ("fp8e4m3",)


def test_e8m0_decode_matches_torch():
    e = np.arange(256)
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).float().numpy()
    ours = O.e8m0_decode(e)
    assert np.array_equal(ours[:255], ref[:255]) and np.isnan(ours[255]) and np.isnan(ref[255])
    assert O.e8m0_decode(np.array([127]))[0] == 1.0


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, 1.0039062, 1.0117188, 3.4e38, -3.4e38, 1e-40, np.inf, -np.inf], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_round(x), ref)


@pytest.mark.parametrize("target", ["fp8e4m3", "fp8e5m2"])
def test_fp8_round_in_range_matches_torch(target):
    rng = np.random.default_rng(4)
    vmax = O.FP8_SPECS[target][2]
    x = rng.uniform(-vmax, vmax, 3000).astype(np.float32)
    x[:200] = rng.standard_normal(200).astype(np.float32) * 1e-3
    tt = {"fp8e4m3": torch.float8_e4m3fn, "fp8e5m2": torch.float8_e5m2}[target]
    ref = torch.from_numpy(x).to(tt).view(torch.uint8).numpy()
    assert np.array_equal(O.fp8_round(x, target), ref)


# ----------------------------------------------------------------------------- packer
@pytest.mark.parametrize("bits", [4, 6])
@pytest.mark.parametrize("count", [1, 7, 8, 33, 250])
def test_pack_codes_matches_both_reference_packers(bits, count):
    """np.packbits LSB-first (benchmark_dtypes.py:150-152) and the big-integer packer
    (test_packed.py:81-84) agree with pack_codes, including the zero-padded tail."""
    codes = np.random.default_rng(count).integers(0, 1 << bits, count).astype(np.uint8)
    ours = O.pack_codes(codes, bits)
    assert ours.tolist() == O.payload_bytes(codes.tolist(), bits)
    shifts = np.arange(bits, dtype=np.uint8)
    packbits = np.packbits(((codes[:, None] >> shifts) & 1).reshape(-1), bitorder="little")
    assert np.array_equal(ours, packbits)
    assert np.array_equal(O.payloads(ours, "uint4" if bits == 4 else "fp6_e2m3", count), codes)


# ----------------------------------------------------------------------------- quantiser
@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
def test_quantize_mx_is_nearest_code_ties_to_even(fmt):
    """Brute force: every element's code is the arg-min distance code (ties -> even
    mantissa LSB); the scale exponent is floor(log2(amax)) - emax_elem."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 96)).astype(np.float32) * np.float32(0.02)
    x[0, :32] = 0.0
    x[1, 5] = 1e-30
    codes, e = O.quantize_mx(x, fmt, 32)
    table = O.code_table(fmt).astype(np.float64)
    bits = O.bits_of(fmt)
    for r in range(x.shape[0]):
        for b in range(3):
            blk = x[r, 32 * b:32 * b + 32].astype(np.float64)
            amax = np.abs(blk).max()
            exp = (math.frexp(amax)[1] - 1 - O.EMAX_ELEM[fmt]) if amax > 0 else 0
            assert int(e[r, b]) - 127 == max(-127, min(127, exp))
            for j, v in enumerate(blk / 2.0 ** exp):
                vv = max(min(v, table.max()), -table.max())
                d = np.abs(table - vv)
                best = [int(c) for c in np.flatnonzero(d == d.min())]
                if len(best) > 1:
                    best = [c for c in best if c & 1 == 0] or best
                    mags = {c & ((1 << (bits - 1)) - 1) for c in best}
                    assert (int(codes[r, 32 * b + j]) & ((1 << (bits - 1)) - 1)) in mags
                else:
                    c = int(codes[r, 32 * b + j])
                    assert table[c] == table[best[0]]


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
def test_quantize_mx_exact_values_round_trip(fmt):
    """Values already on the grid (with the block's amax at the top binade) survive."""
    rng = np.random.default_rng(6)
    table = O.code_table(fmt)
    codes = rng.integers(0, table.size, (4, 64)).astype(np.uint8)
    codes[:, ::32] = table.size // 2 - 1  # largest magnitude in every block fixes the exponent
    exps = rng.integers(-5, 5, (4, 2))
    vals = table[codes] * np.repeat(2.0 ** exps, 32, axis=1)
    q, e = O.quantize_mx(vals.astype(np.float32), fmt, 32)
    back = O.dequant_f64(O.pack_codes(q, O.bits_of(fmt)), fmt, (4, 64), O.e8m0_decode(e), 32)
    assert np.array_equal(back, vals)


# ----------------------------------------------------------------------------- C restatement
@pytest.fixture(scope="module")
def oracle_lib():
    if not ORACLE_LIB.exists():
        pytest.skip("oracle/liboracle_cpu.so not built (make -C oracle)")
    return ctypes.CDLL(str(ORACLE_LIB))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.parametrize("fmt", list(O.FORMATS))
@pytest.mark.parametrize("k", [70, 71])  # 4-bit codes: the two-per-byte path, then the bit-addressed one
def test_c_dequant_matches_numpy_oracle(oracle_lib, fmt, k):
    rng = np.random.default_rng(7)
    n, bs = 5, 32
    bits = O.bits_of(fmt)
    data = rng.integers(0, 256, (n * k * bits + 7) // 8).astype(np.uint8)
    scales = rng.uniform(0.005, 0.02, (n, 3)).astype(np.float16).astype(np.float32)
    ref = O.unpack(data, fmt, (n, k), scales, bs)
    out = np.empty((n, k), np.float32)
    oracle_lib.oracle_dequant_f32(_p(data), ctypes.c_int64(data.size), FMT_IDS[fmt], ctypes.c_int64(n),
                                  ctypes.c_int64(k), _p(scales), ctypes.c_int64(bs), _p(out))
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("k", [5, 300])  # shorter than the 16 partial sums; 18 full rounds and a tail
def test_c_linear_and_rounding(oracle_lib, k):
    rng = np.random.default_rng(8)
    m, n = 3, 17
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = np.empty((m, n), np.float32)
    oracle_lib.oracle_linear_f32(_p(w), _p(x), ctypes.c_int64(m), ctypes.c_int64(n), ctypes.c_int64(k), _p(y))
    assert O.max_rel_err(y, O.matmul_reference(x, w.T)) < 1e-4
    h = np.empty(y.size, np.uint16)
    oracle_lib.oracle_round_bf16(_p(y), ctypes.c_int64(y.size), _p(h))
    assert np.array_equal(h, O.bf16_round(y).reshape(-1))
    oracle_lib.oracle_round_f16(_p(y), ctypes.c_int64(y.size), _p(h))
    assert np.array_equal(h, y.astype(np.float16).view(np.uint16).reshape(-1))


def test_max_rel_err_detects_a_wrong_element():
    e = np.linspace(-1, 1, 101)
    a = e.copy()
    a[17] *= 1.05
    assert O.max_rel_err(a, e) > 0.04 and O.max_rel_err(e, e) == 0.0


# ----------------------------------------------------------------------------- fixtures
def test_oracle_reproduces_committed_fixture():
    """Regression pin: the oracle still produces the committed seeded vectors."""
    path = Path(__file__).parent / "golden" / "oracle_fixtures.npz"
    fx = np.load(path)
    for fmt in ("int4", "fp4_e2m1", "fp6_e2m3", "fp6_e3m2"):
        data = fx[f"{fmt}_data"]
        scales = fx[f"{fmt}_scales"]
        shape = tuple(fx[f"{fmt}_shape"])
        deq = O.unpack(data, fmt, shape, O.e8m0_decode(scales) if fmt != "int4" else scales.astype(np.float32), 32)
        assert np.array_equal(deq.view(np.uint32), fx[f"{fmt}_deq"].view(np.uint32))
    codes, e = O.quantize_mx(fx["quant_x"], "fp4_e2m1", 32)
    assert np.array_equal(codes, fx["quant_codes"]) and np.array_equal(e, fx["quant_e"])
