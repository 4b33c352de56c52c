"""GPU parity of decode, pack and quantise (gfx950 kernels through the C ABI) vs the oracle.

Bit-exact bar: every decoded value is compared as raw bits, so -0.0 and rounding
of bf16/fp16/fp8 results count.
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import packed_oracle as O
from tinygrad_mi355x.codegen.decomp.mi355x import FORMATS, PackedTensor, pack, quantize_mx

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
DT_NAMES = {torch.float32: "float32", torch.float64: "float64", torch.float16: "float16", torch.bfloat16: "bfloat16",
            torch.int32: "int32", torch.int64: "int64", torch.int8: "int8", torch.uint8: "uint8",
            torch.float8_e4m3fn: "fp8e4m3", torch.float8_e5m2: "fp8e5m2"}


def bits_of(t: torch.Tensor) -> np.ndarray:
    """Raw bit patterns of a device tensor as an unsigned numpy array."""
    t = t.detach().cpu().contiguous()
    view = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
    arr = t.view(view).numpy()
    return arr.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[t.element_size()])


def oracle_bits(values: np.ndarray, dt: torch.dtype) -> np.ndarray:
    if dt in (torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2) or values.dtype == np.uint8:
        return values.astype({2: np.uint16, 1: np.uint8}[torch.empty((), dtype=dt).element_size()])
    return values.view({2: np.uint16, 4: np.uint32, 8: np.uint64}[values.itemsize])


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
def test_complete_ocp_payloads(dev, fmt):
    """test_packed.py:87-101 on the device: all payloads, both zeros, bit-exact."""
    positive = GOLDEN["golden_positive_values"]["values"][fmt]
    bits = 4 if fmt.startswith("fp4") else 6
    data = torch.tensor(O.payload_bytes(list(range(1 << bits)), bits), dtype=torch.uint8, device=dev)
    actual = PackedTensor(data, fmt, (1 << bits,)).unpack()
    assert actual.dtype is torch.float32
    assert actual.tolist() == [*positive, *[-x for x in positive]]
    assert math.copysign(1, actual[len(positive)].item()) == -1


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
def test_integer_nibbles(dev, fmt):
    data = torch.tensor(O.payload_bytes(list(range(16)), 4), dtype=torch.uint8, device=dev)
    out = PackedTensor(data, fmt, (16,)).unpack()
    assert out.dtype is torch.int32 and out.tolist() == GOLDEN["integer_nibbles"][fmt]


def test_readme_uint4(dev):
    case = GOLDEN["readme_uint4"]
    packed = PackedTensor(torch.tensor(case["data"], dtype=torch.uint8, device=dev), "uint4", tuple(case["shape"]))
    assert packed.unpack().tolist() == case["unpacked"]


def test_double_block_scales(dev):
    case = GOLDEN["double_block_scales"]
    packed = PackedTensor(torch.tensor(case["data"], dtype=torch.uint8, device=dev), case["format"], tuple(case["shape"]),
                          torch.tensor(case["scales"], dtype=torch.float64, device=dev), block_size=case["block_size"])
    decoded = packed.unpack()
    assert decoded.dtype is torch.float64 and decoded.tolist() == case["decoded"]


@pytest.mark.parametrize("case", GOLDEN["large_bit_positions"]["cases"])
def test_large_packed_bit_positions(dev, case):
    """Decode across the signed 32-bit bit and element offsets (test_packed.py:147-174)."""
    fmt, kind, scaled = case
    pattern = GOLDEN["large_bit_positions"]["pattern"]
    bits = 4 if fmt == "uint4" else 6
    boundary = 2 ** 31 // bits if kind == "bit" else 2 ** 31
    count = boundary + 32
    byte_count = (count * bits + 7) // 8
    storage = torch.tensor(pattern, dtype=torch.uint8, device=dev).repeat((byte_count + 16) // 17)[:byte_count]
    scales = None
    if scaled:
        scale_count = (count + 31) // 32
        scales = torch.tensor(GOLDEN["large_bit_positions"]["scales"], dtype=torch.float32, device=dev)
        scales = scales.repeat((scale_count + 2) // 3)[:scale_count]
    result = PackedTensor(storage, fmt, (count,), scales).unpack()[boundary - 3:boundary + 7].cpu().tolist()
    del storage
    torch.cuda.empty_cache()
    expected = []
    golden = GOLDEN["golden_positive_values"]["values"]
    for index in range(boundary - 3, boundary + 7):
        payload = O.payload_at(lambda j: pattern[j % 17], index, bits)
        value = payload if fmt == "uint4" else golden[fmt][payload & 31] * (-1 if payload & 32 else 1)
        expected.append(value * (GOLDEN["large_bit_positions"]["scales"][index // 32 % 3] if scaled else 1))
    assert result == expected


@pytest.mark.parametrize("fmt", list(FORMATS))
@pytest.mark.parametrize("shape", [(3, 70), (4, 128), (1, 33), (257,)])
@pytest.mark.parametrize("scale_dt", [None, torch.float16, torch.float32, torch.float8_e8m0fnu, torch.float64])
def test_unpack_random_bit_exact(dev, fmt, shape, scale_dt):
    rng = np.random.default_rng(hash((fmt, shape, str(scale_dt))) % 2**32)
    count = math.prod(shape)
    bits = FORMATS[fmt][0]
    data = rng.integers(0, 256, (count * bits + 7) // 8 + 3).astype(np.uint8)  # extra bytes are ignored
    bs = 32
    sshape = shape[:-1] + ((shape[-1] + bs - 1) // bs,)
    scales_np = None
    scales = None
    if scale_dt is torch.float8_e8m0fnu:
        e = (127 + rng.integers(-6, 5, sshape)).astype(np.uint8)
        scales = torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu)
        scales_np, sname = O.e8m0_decode(e), "float32"
    elif scale_dt is not None:
        npdt = {torch.float16: np.float16, torch.float32: np.float32, torch.float64: np.float64}[scale_dt]
        scales_np = rng.uniform(0.005, 0.02, sshape).astype(npdt)
        scales = torch.from_numpy(scales_np).to(dev)
        sname = DT_NAMES[scale_dt]
    packed = PackedTensor(torch.from_numpy(data).to(dev), fmt, shape, scales, bs)
    out_dtypes = [None, torch.float32, torch.bfloat16, torch.float16]
    if scale_dt is None:
        out_dtypes += [torch.int32] + ([torch.float8_e4m3fn] if fmt != "int4" and fmt != "uint4" else [])
    for dt in out_dtypes:
        got = packed.unpack(dt)
        want = O.unpack(data, fmt, shape, scales_np, bs, DT_NAMES.get(dt) if dt else None,
                        scale_dtype=sname if scale_dt is not None else None)
        assert got.shape == shape
        assert np.array_equal(bits_of(got).reshape(-1), oracle_bits(np.asarray(want), got.dtype).reshape(-1)), (fmt, dt)


@pytest.mark.parametrize("fmt,target", [(f, t) for f in ("fp4_e2m1", "fp6_e2m3", "fp6_e3m2")
                                        for t in (torch.float8_e4m3fn, torch.float8_e5m2)])
def test_fp8_unpack(dev, fmt, target):
    """Exact FP8 candidates use the direct encode; E2M3 -> E5M2 rounds through the cast path."""
    bits = FORMATS[fmt][0]
    codes = np.arange(1 << bits, dtype=np.uint8)
    data = torch.from_numpy(O.pack_codes(codes, bits)).to(dev)
    got = PackedTensor(data, fmt, (codes.size,)).unpack(target)
    assert got.dtype is target
    ref = torch.from_numpy(O.decode_values(codes, fmt)).to(target).view(torch.uint8).numpy()
    assert np.array_equal(bits_of(got), ref)


@pytest.mark.parametrize("bits,fmt", [(4, "uint4"), (6, "fp6_e3m2")])
@pytest.mark.parametrize("count", [1, 9, 1000, 4099])
def test_pack_codes_device(dev, bits, fmt, count):
    codes = np.random.default_rng(count).integers(0, 1 << bits, count).astype(np.uint8)
    packed = pack(torch.from_numpy(codes).to(dev), fmt)
    assert packed.data.cpu().numpy().tolist() == O.pack_codes(codes, bits).tolist()


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_quantize_mx_device(dev, fmt, xdt):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((33, 256)) * 0.02).astype(np.float32)
    x[0, :32] = 0
    xt = torch.from_numpy(x).to(dev).to(xdt)
    q = quantize_mx(xt, fmt, 32)
    assert q.scales.dtype is torch.float8_e8m0fnu
    codes, e = O.quantize_mx(xt.float().cpu().numpy(), fmt, 32)
    assert np.array_equal(q.scales.view(torch.uint8).cpu().numpy(), e)
    assert np.array_equal(q.data.cpu().numpy(), O.pack_codes(codes, FORMATS[fmt][0]))


def test_bf16_rounding_instruction_on_every_fp32_pattern(dev):
    """The bf16 epilogues round with one v_cvt_pk_bf16_f32 per pair; it must equal integer
    round-to-nearest-even (NaN -> quiet NaN) on all 2^32 patterns, in both halves of the pair."""
    from tinygrad_mi355x.runtime import kernels as K

    lib = K.load_library()
    bad = torch.tensor([0, -1], dtype=torch.int32, device=dev)
    K.check("tgm_probe_bf16_rounding", lib.tgm_probe_bf16_rounding(0, 1 << 32, None, bad.data_ptr(), K.stream_of(bad)))
    n, low = bad.cpu().numpy().view(np.uint32)
    assert n == 0, f"{n} mismatches, first at {low:#010x}"


@pytest.mark.parametrize("first", [0x00000000, 0x007F0000, 0x3F7F0000, 0x7F7F0000, 0x7F800000, 0x7FBE0000,
                                   0x80000000, 0xFF7F0000, 0xFFFE0000])
def test_bf16_rounding_instruction_against_the_oracle(dev, first):
    """Zeros and subnormals, the 1.0 boundary, overflow to infinity, infinities, signalling and
    quiet NaNs of both signs: the written bf16 bits equal the oracle's rounding bit for bit."""
    from tinygrad_mi355x.runtime import kernels as K

    count = 1 << 17
    lib = K.load_library()
    bits = torch.empty(count, dtype=torch.int16, device=dev)
    bad = torch.tensor([0, -1], dtype=torch.int32, device=dev)
    K.check("tgm_probe_bf16_rounding", lib.tgm_probe_bf16_rounding(first, count, bits.data_ptr(), bad.data_ptr(),
                                                                   K.stream_of(bits)))
    x = np.arange(first, first + count, dtype=np.uint64).astype(np.uint32).view(np.float32)
    assert np.array_equal(bits_of(bits), O.bf16_round(x))
    assert bad.cpu().numpy().view(np.uint32).tolist() == [0, 0xFFFFFFFF]
