"""Packed low-bit tensors: storage record, decode and block-scale API.

Mirrors ``PackedTensor`` of alexandreteles/tinygrad-dx12
(src/tinygrad_dx12/codegen/decomp/dx12.py:14-149) over torch tensors: the same
constructor, validation messages, default dtypes, FP8 shortcut and intermediate
selection.  Decoding runs in the gfx950 kernel ``tgm_unpack``; there is no host
implementation.

Extensions (no reference counterpart, the reference only takes pre-packed bytes,
dx12.py:26-30): :func:`pack` packs payload codes with the same LSB-first stream as
the reference harness (scripts/benchmark_dtypes.py:129-152) and :func:`quantize_mx`
quantises a tensor to an MX format with E8M0 block scales held as
``torch.float8_e8m0fnu`` (numeric scales 2**(e-127), so they satisfy dx12.py:20-23).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from tinygrad_mi355x import dtype as D
from tinygrad_mi355x.codegen.decomp.formats import FORMATS, MX_FORMATS  # noqa: F401  (dx12.py:10)
from tinygrad_mi355x.codegen.program import unpack_program
from tinygrad_mi355x.runtime import kernels as K

# Exact unscaled FP8 destinations (dx12.py:11).
FP8_CANDIDATES = {
    "fp4_e2m1": (torch.float8_e4m3fn, torch.float8_e5m2),
    "fp6_e2m3": (torch.float8_e4m3fn,),
    "fp6_e3m2": (torch.float8_e4m3fn, torch.float8_e5m2),
}


@dataclass(frozen=True)
class PackedTensor:
    """Packed low-bit weights on the HIP device (dx12.py:14-47).

    ``data`` is one flat uint8 device tensor holding every code of the row-major
    ``shape`` back to back as a bit stream, lowest bits first: two 4-bit codes per byte,
    four 6-bit codes per three bytes (a 6-bit code can cross a byte boundary).  The FP4
    and FP6 codes are the OCP formats without infinities or NaNs.  ``scales``, when
    given, hold one factor per ``block_size`` consecutive codes along the last axis
    (shape ``shape[:-1] + (ceil(K / block_size),)``), in any numeric dtype; E8M0 bytes
    (``torch.float8_e8m0fnu``) are OCP MX shared exponents.
    """

    data: torch.Tensor
    format: str
    shape: tuple[int, ...]
    scales: torch.Tensor | None = None
    block_size: int = 32

    def __post_init__(self) -> None:
        """Reject missing format metadata, insufficient storage and incompatible scales (dx12.py:32-47)."""
        object.__setattr__(self, "shape", tuple(int(x) for x in self.shape))
        if self.format not in FORMATS:
            raise ValueError(f"unknown packed format {self.format!r}")
        if not self.shape or any(x < 0 for x in self.shape):
            raise ValueError("packed shape must contain nonnegative dimensions")
        if not isinstance(self.data, torch.Tensor) or self.data.dtype is not torch.uint8 or self.data.dim() != 1:
            raise ValueError("packed data must be a flat uint8 Tensor")
        if self.data.numel() < (math.prod(self.shape) * FORMATS[self.format][0] + 7) // 8:
            raise ValueError("packed storage is smaller than the declared shape")
        if self.block_size < 1:
            raise ValueError("packed block size must be positive")
        if self.scales is not None:
            expected = self.shape[:-1] + ((self.shape[-1] + self.block_size - 1) // self.block_size,)
            if tuple(self.scales.shape) != expected or self.scales.device != self.data.device:
                raise ValueError("packed scales have incompatible shape or device")

    @property
    def device(self) -> torch.device:
        return self.data.device

    def desc(self, data: torch.Tensor | None = None, scales: torch.Tensor | None = None):
        """The kernel programs' view of this operand (``codegen/program.PackedDesc``), for the
        given contiguous storage (default: this record's)."""
        from tinygrad_mi355x.codegen.program import PackedDesc

        data = self.data if data is None else data
        scales = self.scales if scales is None else scales
        return PackedDesc(self.format, self.shape, data.numel(), None if scales is None else scales.data_ptr(),
                          None if scales is None else str(scales.dtype).rsplit(".", 1)[-1], self.block_size)

    @property
    def bits(self) -> int:
        return FORMATS[self.format][0]

    def default_dtype(self) -> torch.dtype:
        """Unscaled integers decode to int32, unscaled floats to float32, scaled data to at
        least float32 (keeping float64 scales) -- dx12.py:57-64."""
        integer = self.format in ("int4", "uint4")
        if self.scales is not None:
            return D.least_upper_dtype(torch.float32, self.scales.dtype)
        return torch.int32 if integer else torch.float32

    def unpack(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """Decode to numeric elements and apply scales at their K-block boundaries (dx12.py:49-106).

        Multiplication happens in ``least_upper(float32, scales.dtype, dtype)``, then the
        result is cast to ``dtype``.  Unscaled FP4/FP6 decoded to an exact FP8 dtype use the
        direct re-encode.  Runs the gfx950 ``tgm_unpack`` kernel on the data's stream.
        """
        dtype = dtype or self.default_dtype()
        count = math.prod(self.shape)
        if not count:
            return torch.empty(self.shape, dtype=dtype, device=self.data.device)
        K.require_device(self.data)
        data = self.data if self.data.is_contiguous() else self.data.contiguous()
        scales = None
        if self.scales is not None:
            scales = self.scales if self.scales.is_contiguous() else self.scales.contiguous()
        out = torch.empty(self.shape, dtype=dtype, device=self.data.device)
        K.dtype_id(dtype)  # ValueError for dtypes the kernels do not write
        program = unpack_program(self.desc(data, scales), str(dtype).rsplit(".", 1)[-1])
        program.launch(out.data_ptr(), data.data_ptr(), 0, K.stream_of(self.data))
        return out

    def matmul(self, other: torch.Tensor | "PackedTensor") -> torch.Tensor:
        """Multiply through the explicit matrix API; these kernels define no gradient (dx12.py:108-112)."""
        from tinygrad_mi355x.codegen.linalg import matmul

        return matmul(self, other)

    # ------------------------------------------------------------------ construction helpers
    @classmethod
    def pack(cls, codes: torch.Tensor, format: str, shape: tuple[int, ...] | None = None,
             scales: torch.Tensor | None = None, block_size: int = 32) -> "PackedTensor":
        return pack(codes, format, shape, scales, block_size)

    @classmethod
    def quantize(cls, x: torch.Tensor, format: str, block_size: int = 32) -> "PackedTensor":
        return quantize_mx(x, format, block_size)


def pack(codes: torch.Tensor, format: str, shape: tuple[int, ...] | None = None,
         scales: torch.Tensor | None = None, block_size: int = 32) -> PackedTensor:
    """Pack payload codes (one per uint8, low ``bits`` bits used) LSB first into a PackedTensor."""
    if format not in FORMATS:
        raise ValueError(f"unknown packed format {format!r}")
    if codes.dtype is not torch.uint8:
        raise ValueError("codes must be a uint8 tensor of payloads")
    K.require_device(codes)
    shape = tuple(codes.shape) if shape is None else tuple(shape)
    flat = codes.reshape(-1).contiguous()
    if flat.numel() != math.prod(shape):
        raise ValueError("code count does not match the packed shape")
    bits = FORMATS[format][0]
    out = torch.empty((flat.numel() * bits + 7) // 8, dtype=torch.uint8, device=codes.device)
    K.call("tgm_pack_codes", flat.data_ptr(), flat.numel(), bits, out.data_ptr(), K.stream_of(codes))
    return PackedTensor(out, format, shape, scales, block_size)


def unpack(packed: PackedTensor, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Functional form of ``PackedTensor.unpack``: the node a traced program records for a decode
    (tinygrad_mi355x.codegen.matmul rewrites products whose operand it is)."""
    return packed.unpack(dtype)


def quantize_mx(x: torch.Tensor, format: str, block_size: int = 32) -> PackedTensor:
    """MX-quantise ``x`` [..., K] along its last axis into ``format`` with E8M0 block scales.

    Shared exponent per block: floor(log2(amax)) - emax_elem (E2M1/E2M3: 2, E3M2: 4),
    clamped to [-127, 127]; all-zero blocks use 2**0.  Elements are rounded to the
    nearest code with ties to the even payload and saturate at the largest finite value.
    """
    if format not in MX_FORMATS:
        raise ValueError(f"MX quantisation needs one of {MX_FORMATS}, got {format!r}")
    if x.dim() < 1 or x.shape[-1] < 1:
        raise ValueError("quantize_mx needs a tensor with a nonempty last dimension")
    K.require_device(x)
    shape = tuple(x.shape)
    k = shape[-1]
    rows = math.prod(shape[:-1])
    src = x.contiguous()
    bits = FORMATS[format][0]
    nblk = (k + block_size - 1) // block_size
    data = torch.empty((rows * k * bits + 7) // 8, dtype=torch.uint8, device=x.device)
    scales = torch.empty(shape[:-1] + (nblk,), dtype=torch.uint8, device=x.device)
    K.call("tgm_quantize_mx", src.data_ptr(), K.dtype_id(src.dtype), rows, k, K.FORMAT_IDS[format], block_size,
           data.data_ptr(), scales.data_ptr(), K.stream_of(x))
    return PackedTensor(data, format, shape, scales.view(torch.float8_e8m0fnu), block_size)


def matrix_intermediate(a: torch.Tensor | PackedTensor, b: torch.Tensor | PackedTensor, native16: bool = False) -> torch.dtype:
    """Exact common representation of two matrix operands (dx12.py:115-138).

    A common FP8 wins when every packed operand is unscaled with an exact FP8 choice and
    every ordinary operand already has that dtype (E4M3FN before E5M2).  Otherwise the
    declared types are promoted: ordinary dtype; int8/uint8 for unscaled int4/uint4;
    float16 for unscaled FP4/FP6; at least float32 for scaled data.  ``native16`` is kept
    for signature compatibility and does not change the choice.
    """
    sets = []
    for operand in (a, b):
        if isinstance(operand, torch.Tensor):
            sets.append({operand.dtype})
        elif operand.scales is None:
            sets.append(set(FP8_CANDIDATES.get(operand.format, ())))
        else:
            sets.append(set())
    common = set.intersection(*sets)
    for dt in D.FP8:
        if dt in common:
            return dt
    declared = []
    for operand in (a, b):
        if isinstance(operand, torch.Tensor):
            declared.append(operand.dtype)
        elif operand.scales is not None:
            declared.append(D.least_upper_dtype(torch.float32, operand.scales.dtype))
        else:
            declared.append({"int4": torch.int8, "uint4": torch.uint8}.get(operand.format, torch.float16))
    return D.strong_dtype(D.least_upper_dtype(*declared))


def matmul(a: torch.Tensor | PackedTensor, b: torch.Tensor | PackedTensor) -> torch.Tensor:
    """Multiply after decoding packed operands with their default dtypes (dx12.py:141-149).

    The product follows ordinary matmul typing: accumulate in ``sum_acc_dtype`` of the
    promoted dtype; 16-bit and FP8 results are cast back to the promoted dtype.
    """
    from tinygrad_mi355x.codegen.linalg import plain_matmul

    lhs, rhs = [operand.unpack() if isinstance(operand, PackedTensor) else operand for operand in (a, b)]
    if lhs.dim() != 2 or rhs.dim() != 2 or lhs.shape[1] != rhs.shape[0]:
        raise ValueError("matrix operands must have compatible rank-two shapes")
    promoted = D.least_upper_dtype(lhs.dtype, rhs.dtype)
    acc = D.sum_acc_dtype(promoted)
    out = promoted if promoted in (torch.float16, torch.bfloat16, *D.FP8) else acc
    return plain_matmul(lhs, rhs, out, acc)
