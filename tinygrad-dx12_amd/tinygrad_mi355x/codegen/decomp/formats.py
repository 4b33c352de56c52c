"""Packed format table (no torch): ``FORMATS`` of alexandreteles/tinygrad-dx12
src/tinygrad_dx12/codegen/decomp/dx12.py:10 -- (total bits, exponent bits, mantissa bits,
exponent bias); integers have no exponent -- and the formats with OCP MX scaling."""

FORMATS = {"int4": (4, 0, 0, 0), "uint4": (4, 0, 0, 0), "fp4_e2m1": (4, 2, 1, 1), "fp6_e2m3": (6, 2, 3, 1),
           "fp6_e3m2": (6, 3, 2, 3)}
MX_FORMATS = ("fp4_e2m1", "fp6_e2m3", "fp6_e3m2")


def packed_nbytes(format: str, count: int) -> int:
    """Bytes of ``count`` packed elements: ceil(count * bits / 8) (dx12.py:40-41)."""
    return (count * FORMATS[format][0] + 7) // 8
