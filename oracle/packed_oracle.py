"""CPU oracle for the packed low-bit matmul path (test infrastructure only).

This module restates, in NumPy, the reference's packed-format semantics so that
the HIP kernels can be checked against it.  It only checks; it is never the thing
measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.

Reference anchors (paths under ``src/tinygrad_dx12/`` of alexandreteles/tinygrad-dx12):

* ``FORMATS`` / ``FP8_CANDIDATES``            -> codegen/decomp/dx12.py:9-11
* ``payloads`` (bit-stream extraction)        -> codegen/decomp/dx12.py:69-77
* ``fp8_direct`` (unscaled FP8 re-encode)     -> codegen/decomp/dx12.py:78-92
* ``decode_values`` (int / float decode)      -> codegen/decomp/dx12.py:93-100
* ``unpack`` (scale broadcast, multiply, cast)-> codegen/decomp/dx12.py:49-68, 101-106
* ``pack_codes`` (LSB-first packer)           -> scripts/benchmark_dtypes.py:129-152,
                                                 test/backend/test_packed.py:81-84
* ``matmul_reference`` (CPU branch)           -> codegen/linalg.py:169-174

Functions with no reference counterpart, pinned by mathematics instead:

* ``e8m0_decode``   -- OCP MX v1.0 closed form 2**(e-127), e=255 is NaN; also checked
                       against ``torch.float8_e8m0fnu`` in the tests.
* ``quantize_mx``   -- OCP MX shared-exponent choice + round-to-nearest-even element
                       quantisation; pinned by brute-force nearest-code search.
* ``bf16_round`` / ``fp8_round`` -- RNE casts; pinned against torch casts and brute force.

Pinning status of every function is recorded in the tests that exercise it.
"""

from __future__ import annotations

import math

import numpy as np

# (total bits, exponent bits, mantissa bits, exponent bias) -- dx12.py:10
FORMATS = {
    "int4": (4, 0, 0, 0),
    "uint4": (4, 0, 0, 0),
    "fp4_e2m1": (4, 2, 1, 1),
    "fp6_e2m3": (6, 2, 3, 1),
    "fp6_e3m2": (6, 3, 2, 3),
}
# Exact unscaled FP8 destinations per source format -- dx12.py:11
FP8_CANDIDATES = {
    "fp4_e2m1": ("fp8e4m3", "fp8e5m2"),
    "fp6_e2m3": ("fp8e4m3",),
    "fp6_e3m2": ("fp8e4m3", "fp8e5m2"),
}
# (mantissa bits, bias, max finite) of the FP8 targets; E4M3FN has no infinities.
FP8_SPECS = {"fp8e4m3": (3, 7, 448.0), "fp8e5m2": (2, 15, 57344.0)}
# Largest-normal exponent of each element format (OCP MX emax_elem).
EMAX_ELEM = {"fp4_e2m1": 2, "fp6_e2m3": 2, "fp6_e3m2": 4}


def bits_of(fmt: str) -> int:
    return FORMATS[fmt][0]


def packed_nbytes(count: int, fmt: str) -> int:
    """Minimum storage in bytes for ``count`` elements (dx12.py:40)."""
    return (count * bits_of(fmt) + 7) // 8


# --------------------------------------------------------------------------- bit stream
def payloads(data: np.ndarray, fmt: str, count: int) -> np.ndarray:
    """Extract ``count`` raw payloads from a flat uint8 array (dx12.py:69-77).

    Groups of ``bits/2`` bytes form one little-endian word holding four payloads;
    payload ``i`` of a word is ``(word >> i*bits) & mask``.
    """
    bits = bits_of(fmt)
    group = bits // 2
    flat = np.asarray(data, dtype=np.uint8).reshape(-1)
    padded = np.concatenate([flat, np.zeros((-flat.size) % group, dtype=np.uint8)]).reshape(-1, group)
    word = np.zeros(padded.shape[0], dtype=np.uint32)
    for i in range(group):
        word |= padded[:, i].astype(np.uint32) << np.uint32(8 * i)
    shifts = (np.arange(4, dtype=np.uint32) * np.uint32(bits))[None, :]
    out = (word[:, None] >> shifts) & np.uint32((1 << bits) - 1)
    return out.reshape(-1)[:count]


def payload_at(pattern_byte, index: int, bits: int) -> int:
    """Closed-form payload of element ``index`` (test_packed.py:168-173 formula).

    ``pattern_byte(j)`` returns storage byte ``j``.
    """
    byte, shift = divmod(index * bits, 8)
    return ((pattern_byte(byte) | pattern_byte(byte + 1) << 8) >> shift) & ((1 << bits) - 1)


# --------------------------------------------------------------------------- decoding
def decode_values(p: np.ndarray, fmt: str) -> np.ndarray:
    """Numeric value of each payload (dx12.py:93-100): int32 for integers, fp32 for floats."""
    bits, _, man, bias = FORMATS[fmt]
    p = np.asarray(p, dtype=np.uint32)
    if fmt == "int4":
        return ((p.astype(np.int32) ^ 8) - 8).astype(np.int32)
    if fmt == "uint4":
        return p.astype(np.int32)
    frac = (p & np.uint32((1 << man) - 1)).astype(np.float32)
    exp = ((p >> np.uint32(man)) & np.uint32((1 << (bits - man - 1)) - 1)).astype(np.int32)
    sig = np.where(exp == 0, frac, frac + np.float32(1 << man)).astype(np.float32)
    power = np.exp2((np.where(exp == 0, 1, exp) - bias - man).astype(np.float32)).astype(np.float32)
    val = (sig * power).astype(np.float32)
    neg = (p & np.uint32(1 << (bits - 1))) != 0
    return np.where(neg, -val, val).astype(np.float32)


def fp8_direct(p: np.ndarray, fmt: str, target: str) -> np.ndarray:
    """Re-encode unscaled FP4/FP6 payloads as FP8 bytes (dx12.py:78-92)."""
    bits, _, man, bias = FORMATS[fmt]
    t_man, t_bias, _ = FP8_SPECS[target]
    p = np.asarray(p, dtype=np.int64)
    fraction = p & ((1 << man) - 1)
    exponent = (p >> man) & ((1 << (bits - man - 1)) - 1)
    subnormal = np.zeros_like(p)
    for high in range(man):
        encoded = ((t_bias + 1 - bias - man + high) << t_man) | ((fraction << (t_man - high)) & ((1 << t_man) - 1))
        subnormal = np.where(fraction >= (1 << high), encoded, subnormal)
    normal = ((exponent + t_bias - bias) << t_man) | (fraction << (t_man - man))
    encoded = ((p >> (bits - 1)) << 7) | np.where(exponent == 0, subnormal, normal)
    return encoded.astype(np.uint8)


def fp8_decode(b: np.ndarray, target: str) -> np.ndarray:
    """Value of FP8 bytes (OCP E4M3FN: 0x7F/0xFF NaN, no inf; E5M2: IEEE-like)."""
    t_man, t_bias, _ = FP8_SPECS[target]
    b = np.asarray(b, dtype=np.int64)
    e_bits = 7 - t_man
    frac = b & ((1 << t_man) - 1)
    exp = (b >> t_man) & ((1 << e_bits) - 1)
    val = np.where(exp == 0, frac * 2.0 ** (1 - t_bias - t_man), (frac + (1 << t_man)) * np.exp2(exp - t_bias - t_man))
    if target == "fp8e4m3":
        val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    else:
        val = np.where((exp == 31) & (frac == 0), np.inf, np.where(exp == 31, np.nan, val))
    return np.where(b & 0x80, -val, val).astype(np.float32)


# --------------------------------------------------------------------------- rounding
def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bfloat16 with round-to-nearest-even; returns uint16 bit patterns."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = np.where(nan, (u >> 16) | 0x40, rounded)
    return out.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def fp8_round(x: np.ndarray, target: str) -> np.ndarray:
    """Round to the nearest FP8 value, ties to even, saturating to +-max finite.

    NaN maps to the format's NaN.  Brute force over the 256 encodings, so only
    suitable for test-sized inputs.
    """
    x = np.asarray(x, dtype=np.float64).reshape(-1)
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8_decode(codes, target).astype(np.float64)
    finite = np.isfinite(vals)
    _, _, vmax = FP8_SPECS[target]
    out = np.empty(x.size, dtype=np.uint8)
    fc, fv = codes[finite], vals[finite]
    for i, v in enumerate(x):
        if math.isnan(v):
            out[i] = 0x7F if target == "fp8e4m3" else 0x7E
            continue
        c = min(max(v, -vmax), vmax)
        d = np.abs(fv - c)
        best = np.flatnonzero(d == d.min())
        if len(best) > 1:  # tie: prefer even mantissa LSB, and keep the sign of zero
            even = [j for j in best if (fc[j] & 1) == 0]
            best = even or list(best)
            signed = [j for j in best if (fc[j] >> 7) == (1 if math.copysign(1, v) < 0 else 0)]
            best = signed or best
        out[i] = fc[best[0]]
    return out


# --------------------------------------------------------------------------- scales
def e8m0_decode(e: np.ndarray) -> np.ndarray:
    """OCP MX E8M0 scale: 2**(e-127); 255 is NaN (no reference counterpart)."""
    e = np.asarray(e, dtype=np.int64)
    val = np.ldexp(np.float64(1.0), (np.minimum(e, 254) - 127).astype(np.int64)).astype(np.float32)
    return np.where(e == 255, np.float32(np.nan), val).astype(np.float32)


def scale_dtype_for(scale_dtype: str | None, dtype: str) -> str:
    """Multiplication precision least_upper(fp32, scale, dtype) (dx12.py:103).

    Within this path that is fp64 when either side is fp64, else fp32.
    """
    return "float64" if "float64" in (scale_dtype, dtype) else "float32"


# --------------------------------------------------------------------------- unpack
NUMPY_TYPES = {
    "bool": np.bool_, "int8": np.int8, "uint8": np.uint8, "int16": np.int16, "uint16": np.uint16,
    "int32": np.int32, "uint32": np.uint32, "int64": np.int64, "uint64": np.uint64,
    "float16": np.float16, "float32": np.float32, "float64": np.float64,
}


def cast_to(values: np.ndarray, dtype: str) -> np.ndarray:
    """Final ``.cast(dtype)`` of dx12.py:106.  bf16/fp8 are returned as raw bit patterns."""
    if dtype == "bfloat16":
        return bf16_round(values.astype(np.float32))
    if dtype in FP8_SPECS:
        return fp8_round(values, dtype)
    if dtype in ("int8", "uint8", "int16", "uint16", "int32", "uint32", "int64", "uint64") and values.dtype.kind == "f":
        return np.trunc(values).astype(NUMPY_TYPES[dtype])
    return values.astype(NUMPY_TYPES[dtype])


def default_unpack_dtype(fmt: str, scale_dtype: str | None) -> str:
    """Default decode dtype (dx12.py:57-64)."""
    if scale_dtype is not None:
        return "float64" if scale_dtype == "float64" else "float32"
    return "int32" if fmt in ("int4", "uint4") else "float32"


def unpack(data, fmt: str, shape, scales=None, block_size: int = 32, dtype: str | None = None,
           scale_dtype: str | None = None) -> np.ndarray:
    """Decode packed bytes to numbers (dx12.py:49-106).

    ``scales`` is a numeric array of shape ``shape[:-1] + (ceil(K/block),)`` whose
    element type is named by ``scale_dtype`` (defaults to the array's own dtype).
    Returns values in ``dtype``; bfloat16 and fp8 come back as raw bit patterns.
    """
    shape = tuple(shape)
    count = math.prod(shape)
    if scales is not None and scale_dtype is None:
        scale_dtype = {np.float16: "float16", np.float32: "float32", np.float64: "float64"}.get(
            np.asarray(scales).dtype.type, "float32")
    dtype = dtype or default_unpack_dtype(fmt, scale_dtype if scales is not None else None)
    p = payloads(data, fmt, count)
    if scales is None and dtype in FP8_CANDIDATES.get(fmt, ()):
        return fp8_direct(p, fmt, dtype).reshape(shape)
    value = decode_values(p, fmt).reshape(shape)
    if scales is not None:
        sd = scale_dtype_for(scale_dtype, dtype)
        npt = NUMPY_TYPES[sd]
        k = shape[-1]
        sc = np.repeat(np.asarray(scales), block_size, axis=-1)[..., :k]
        value = value.astype(npt) * sc.astype(npt)
    return cast_to(value, dtype)


def dequant_f64(data, fmt: str, shape, scales=None, block_size: int = 32) -> np.ndarray:
    """Exact dequantised values as float64 (code * scale; exact for every format here)."""
    shape = tuple(shape)
    value = decode_values(payloads(data, fmt, math.prod(shape)), fmt).astype(np.float64).reshape(shape)
    if scales is not None:
        value = value * np.repeat(np.asarray(scales, dtype=np.float64), block_size, axis=-1)[..., : shape[-1]]
    return value


# --------------------------------------------------------------------------- packing
def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack payload codes least-significant bit first, zero-padded tail.

    Same byte stream as ``np.packbits(bits, bitorder="little")`` over the codes'
    low ``bits`` bits (benchmark_dtypes.py:150-152, test_packed.py:81-84).
    """
    c = np.asarray(codes, dtype=np.uint32).reshape(-1)
    if bits == 4:
        if c.size % 2:
            c = np.concatenate([c, np.zeros(1, np.uint32)])
        return ((c[0::2] & 0xF) | ((c[1::2] & 0xF) << 4)).astype(np.uint8)
    shifts = np.arange(bits, dtype=np.uint32)
    bitstream = ((c[:, None] >> shifts) & 1).astype(np.uint8).reshape(-1)
    return np.packbits(bitstream, bitorder="little")


def payload_bytes(codes, bits: int) -> list[int]:
    """Big-integer packer restated from test_packed.py:81-84 (for fixtures)."""
    number = sum(int(code) << (i * bits) for i, code in enumerate(codes))
    return list(number.to_bytes((len(codes) * bits + 7) // 8, "little"))


# --------------------------------------------------------------------------- quantiser
def code_table(fmt: str) -> np.ndarray:
    """Value of every payload of a float format, indexed by payload."""
    return decode_values(np.arange(1 << bits_of(fmt), dtype=np.uint32), fmt)


def _round_magnitude(mag: np.ndarray, fmt: str) -> np.ndarray:
    """Map |x| (already scaled, float64) to the magnitude payload, RNE, saturating."""
    bits = bits_of(fmt)
    pos = code_table(fmt)[: 1 << (bits - 1)].astype(np.float64)  # ascending magnitudes
    mids = (pos[:-1] + pos[1:]) / 2
    idx = np.searchsorted(mids, mag, side="left")  # mag <= mids[i] -> i
    # exact ties (mag == mids[i]) resolve to the even payload of {i, i+1}
    tie = (idx < len(mids)) & (mag == mids[np.minimum(idx, len(mids) - 1)])
    idx = np.where(tie & (idx % 2 == 1), idx + 1, idx)
    return np.minimum(idx, len(pos) - 1).astype(np.uint32)


def quantize_mx(x: np.ndarray, fmt: str, block_size: int = 32):
    """MX-quantise ``x`` [..., K] along the last axis (no reference counterpart).

    Shared exponent per block: ``floor(log2(amax)) - emax_elem`` clamped to
    [-127, 127]; an all-zero block gets exponent 0 (E8M0 byte 127).  Elements
    are divided by 2**exp and rounded to nearest (ties to even payload),
    saturating to the largest finite magnitude.  Returns (codes uint8 [..., K],
    e8m0 bytes uint8 [..., ceil(K/block)]).
    """
    x = np.asarray(x, dtype=np.float32)
    k = x.shape[-1]
    nb = -(-k // block_size)
    pad = nb * block_size - k
    xp = np.concatenate([x, np.zeros(x.shape[:-1] + (pad,), np.float32)], axis=-1) if pad else x
    blocks = xp.reshape(x.shape[:-1] + (nb, block_size)).astype(np.float64)
    amax = np.abs(blocks).max(axis=-1)
    with np.errstate(divide="ignore"):
        exp = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1.0))), 0.0)
    # frexp-based floor(log2) avoids log2 rounding at exact powers of two
    m, e = np.frexp(np.where(amax > 0, amax, 1.0))
    exp = np.where(amax > 0, e - 1, 0).astype(np.int64) - EMAX_ELEM[fmt]
    exp = np.where(amax > 0, exp, 0)
    exp = np.clip(exp, -127, 127)
    scaled = blocks / np.ldexp(1.0, exp)[..., None]
    mag = _round_magnitude(np.abs(scaled), fmt)
    sign = (np.signbit(scaled) & (mag > 0)).astype(np.uint32)  # -0 from underflow kept as +0
    codes = (sign << np.uint32(bits_of(fmt) - 1)) | mag
    codes = codes.reshape(xp.shape)[..., :k].astype(np.uint8)
    return codes, (exp + 127).astype(np.uint8)


# --------------------------------------------------------------------------- matmul
def matmul_reference(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Exact-product, wide-accumulate matmul of already-dequantised operands.

    The reference CPU branch (linalg.py:169-174) unpacks to the fp32
    intermediate and reduces with fp32 accumulation; its summation order is
    tinygrad's.  This oracle accumulates in float64 so that every parity check
    measures the kernel's own rounding against a tighter bound.
    """
    return np.asarray(a, dtype=np.float64) @ np.asarray(b, dtype=np.float64)


def max_rel_err(actual: np.ndarray, expected: np.ndarray, floor: float = 1e-3) -> float:
    """Largest elementwise relative error ``|a-e| / max(|e|, floor * max|e|)``.

    The floor keeps outputs that cancel to nearly zero (where any fp32 summation
    order differs in relative terms) from dominating; every other element is
    held to its own relative error.
    """
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    if expected.size == 0:
        return 0.0
    scale = max(float(np.abs(expected).max()), 1e-30)
    denom = np.maximum(np.abs(expected), floor * scale)
    return float((np.abs(actual - expected) / denom).max())
