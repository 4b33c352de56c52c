"""Packed matrix kernels as programs, and the packed path on plugin buffers (no torch).

The reference wraps each LinAlg kernel in a tinygrad PROGRAM with slots (out=0, a=1, b=2), a
launch geometry and ``Estimates(flops=2mnk, bytes=m*n*out + m*k*a + k*n*b)``
(alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/linalg.py:37-58), and runs it with
``custom_kernel`` -> ``Program.__call__`` (:206-218).  ``MatrixProgram`` is that object for the
prebuilt gfx950 kernel library: the same slot order, the family's nominal launch geometry (its
tile grid and workgroup size; the entry point sizes its exact grid), the launch's algorithmic
``Estimates`` and a call on a device stream.  Where the reference counts the decoded operands'
bytes, a packed operand here counts its packed bytes and its scales: that is what the kernel
reads.  The torch adapter (``codegen/linalg.py``) launches these programs with tensor addresses
on torch's stream; ``bench.py`` takes its algorithmic bytes and flops from the same estimates.

The rest of the module is the reference's standalone chain -- ``PackedTensor.matmul`` ->
kernel table -> launch (codegen/decomp/dx12.py:108-112, codegen/linalg.py:136-298) -- over the
plugin's own memory: ``PackedBuffer`` (the PackedTensor record over ``MI355XBuffer`` storage,
with the reference's validation messages), ``Matrix`` (a typed row-major view of a buffer) and
``unpack`` / ``matvec`` / ``matmul_nt``, which allocate results with the device's allocator and
launch on ``MI355XDevice.stream`` under the device lock.  Nothing here imports torch.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable

from tinygrad_mi355x.codegen.decomp.formats import FORMATS, MX_FORMATS, packed_nbytes
from tinygrad_mi355x.renderer.matrix import (GEMM_FP8, GEMM_W, GEMV, GEMV_MAX_ROWS, MatrixKernel, dense_kernel,
                                            mx_kernel)
from tinygrad_mi355x.runtime import library as L
from tinygrad_mi355x.runtime import profile
from tinygrad_mi355x.runtime.support import hip

ACTIVATIONS = ("bfloat16", "float16", "float32")
OUTPUTS = ("bfloat16", "float16", "float32")
FP8 = ("float8_e4m3fn", "float8_e5m2")
SLOTS = ("out", "a", "b")


@dataclass(frozen=True)
class Estimates:
    """Algorithmic work of one launch: ``ops`` arithmetic operations (2 m n k for a product)
    and ``mem`` bytes the kernel must read and write."""

    ops: int
    mem: int


@dataclass(frozen=True)
class PackedDesc:
    """What a program needs of a packed operand: format, logical [N, K] shape, storage bytes
    and the scales (device address, dtype name, block size; no address = unscaled)."""

    format: str
    shape: tuple[int, ...]
    nbytes: int
    scales: int | None = None
    scale_dtype: str | None = None
    block_size: int = 32

    @property
    def scale_bytes(self) -> int:
        if self.scales is None:
            return 0
        blocks = math.prod(self.shape[:-1]) * -(-self.shape[-1] // self.block_size)
        return blocks * L.DTYPE_SIZES[self.scale_dtype]

    @property
    def read_bytes(self) -> int:
        return packed_nbytes(self.format, math.prod(self.shape)) + self.scale_bytes

    def scale_args(self) -> tuple[int | None, int]:
        return (None, -1) if self.scales is None else (self.scales, L.DTYPE_IDS[self.scale_dtype])


class MatrixProgram:
    """One launch of a library kernel: slots (out, a, b), geometry, estimates and the call."""

    slots = SLOTS

    def __init__(self, kernel: MatrixKernel, name: str, groups: int, estimates: Estimates,
                 args: Callable[[int, int, int, int], tuple], slot_bytes: tuple[int, ...] = ()) -> None:
        self.kernel, self.name, self.estimates, self._args = kernel, name, estimates, args
        self.global_size = (max(int(groups), 0), 1, 1)
        self.local_size = (kernel.threads, 1, 1)
        # bytes the kernel reads or writes through each slot (out, a[, b]), from the first
        # element's address: a buffer bound to a slot must hold at least that many
        self.slot_bytes = tuple(max(int(x), 0) for x in slot_bytes)

    def __repr__(self) -> str:
        return f"MatrixProgram({self.name}, groups={self.global_size[0]})"

    def check_slots(self, sizes: tuple[int, ...]) -> None:
        """ValueError unless buffers of ``sizes`` bytes (slot order) cover what the kernel touches."""
        if len(sizes) < len(self.slot_bytes):
            raise ValueError(f"{self.name}: {len(self.slot_bytes)} slot buffers needed, {len(sizes)} given")
        for slot, have, need in zip(SLOTS, sizes, self.slot_bytes):
            if have < need:
                raise ValueError(f"{self.name}: the {slot} buffer holds {have} bytes; the kernel touches {need}")

    def launch(self, out: int, a: int, b: int, stream: int) -> None:
        """Enqueue on ``stream`` with slot addresses (out, a, b); the caller owns ordering."""
        if 0 in self.global_size:
            return
        L.call(self.name, *self._args(out, a, b, stream))

    def __call__(self, out, a, b=None, *, wait: bool = False, timeout: int | None = None) -> float | None:
        """Launch on plugin buffers of one device, on its stream under its lock; seconds when
        ``wait`` (``0.0 if wait else None`` for zero work, as the reference's programs)."""
        bufs = tuple(x for x in (out, a, b) if x is not None)
        dev = out.dev
        if any(x.dev is not dev for x in bufs):
            raise ValueError("MI355X buffer device/signature mismatch")
        self.check_slots(tuple(x.size for x in bufs))
        if 0 in self.global_size:
            return 0.0 if wait else None
        with dev.lock, dev.submitting():
            dev.select()
            start, stop = (hip.event_create(), hip.event_create()) if wait else (0, 0)
            ranged = profile.RangeTiming(dev, self.name) if profile.enabled() else None
            if wait:
                hip.call("hipEventRecord", start, dev.stream)
            self.launch(out.address, a.address, b.address if b is not None else 0, dev.stream)
            if wait:
                hip.call("hipEventRecord", stop, dev.stream)
            if ranged is not None:
                ranged.end(dev)
            dev.submitted(tuple(x.owner for x in bufs), ranged.publish if ranged is not None else None)
        if not wait:
            return None
        try:
            dev.wait_event(stop, timeout, owned=True)
            return hip.elapsed_ms(start, stop) / 1e3
        finally:
            hip.call("hipEventDestroy", start)
            hip.call("hipEventDestroy", stop)


def _extent(rows: int, ld: int, cols: int, dtype: str) -> int:
    """Bytes from the first element to one past the last of a row-major [rows, cols] matrix with
    row stride ``ld`` elements."""
    return 0 if rows <= 0 or cols <= 0 else ((rows - 1) * ld + cols) * L.DTYPE_SIZES[dtype]


def _tiles(rows: int, cols: int, kernel: MatrixKernel) -> int:
    return -(-rows // kernel.tile[0]) * -(-cols // kernel.tile[1])


# ----------------------------------------------------------------------------- program builders
def unpack_program(p: PackedDesc, out_dtype: str) -> MatrixProgram:
    """Decode ``p`` to ``out_dtype`` (slots out, a): PackedTensor.unpack (dx12.py:49-106)."""
    count = math.prod(p.shape)
    est = Estimates(0 if p.scales is None else count, p.read_bytes + count * L.DTYPE_SIZES[out_dtype])
    scales, sdt = p.scale_args()
    fmt, k, odt = L.FORMAT_IDS[p.format], p.shape[-1], L.DTYPE_IDS[out_dtype]
    kernel = MatrixKernel("tgm_unpack", "elementwise", (256, 1, 1), 256)
    return MatrixProgram(kernel, "tgm_unpack", -(-count // 256), est,
                         lambda out, a, b, s: (a, p.nbytes, fmt, count, k, scales, sdt, p.block_size, out, odt, s),
                         (count * L.DTYPE_SIZES[out_dtype], packed_nbytes(p.format, count)))


def weight_program(w: PackedDesc, m: int, x_dtype: str, ldx: int, y_dtype: str, ldy: int) -> MatrixProgram:
    """Y[M, N] = X[M, K] @ deq(W)[N, K]^T (slots out = Y, a = W, b = X): family 1 (GEMV, M <= 16)
    or family 2 (dequant GEMM)."""
    n, k = w.shape
    est = Estimates(2 * m * n * k, w.read_bytes + m * k * L.DTYPE_SIZES[x_dtype] + m * n * L.DTYPE_SIZES[y_dtype])
    scales, sdt = w.scale_args()
    fmt, xdt, ydt = L.FORMAT_IDS[w.format], L.DTYPE_IDS[x_dtype], L.DTYPE_IDS[y_dtype]
    touched = (_extent(m, ldy, n, y_dtype), packed_nbytes(w.format, n * k), _extent(m, ldx, k, x_dtype))
    if m <= GEMV_MAX_ROWS:
        return MatrixProgram(GEMV, "tgm_gemv", _tiles(n, m, GEMV), est,
                             lambda out, a, b, s: (a, fmt, n, k, scales, sdt, w.block_size, b, xdt, m, ldx, out, ydt,
                                                   ldy, s), touched)
    return MatrixProgram(GEMM_W, "tgm_gemm_w", _tiles(n, m, GEMM_W), est,
                         lambda out, a, b, s: (b, xdt, m, ldx, a, fmt, n, k, scales, sdt, w.block_size, out, ydt, ldy,
                                               s), touched)


def mx_program(a: PackedDesc, b: PackedDesc, c_dtype: str, ldc: int) -> MatrixProgram:
    """C[M, N] = deq(A)[M, K] @ deq(B)[N, K]^T for two packed FP4 / FP6 operands (slots out, a, b)."""
    m, k = a.shape
    n = b.shape[0]
    est = Estimates(2 * m * n * k, a.read_bytes + b.read_bytes + m * n * L.DTYPE_SIZES[c_dtype])
    sa, sb = a.scales, b.scales
    fa, fb, cdt = L.FORMAT_IDS[a.format], L.FORMAT_IDS[b.format], L.DTYPE_IDS[c_dtype]
    kernel = mx_kernel(a.format, sa is not None, b.format, sb is not None, k)
    return MatrixProgram(kernel, "tgm_gemm_mx", _tiles(m, n, kernel), est,
                         lambda out, x, y, s: (x, fa, sa, m, y, fb, sb, n, k, out, cdt, ldc, s),
                         (_extent(m, ldc, n, c_dtype), packed_nbytes(a.format, m * k), packed_nbytes(b.format, n * k)))


def dense_program(a_dtype: str, m: int, lda: int, b_dtype: str, n: int, ldb: int, k: int, c_dtype: str, ldc: int,
                  scale_a: int = 0, scale_b: int = 0) -> MatrixProgram:
    """C[M, N] = A[M, K] @ B[N, K]^T for bf16 / f16 pairs or FP8 pairs (slots out, a, b);
    ``scale_a`` / ``scale_b`` are fp32 device scalars (FP8 only, address 0 = none)."""
    est = Estimates(2 * m * n * k, m * k * L.DTYPE_SIZES[a_dtype] + n * k * L.DTYPE_SIZES[b_dtype]
                    + m * n * L.DTYPE_SIZES[c_dtype])
    adt, bdt, cdt = L.DTYPE_IDS[a_dtype], L.DTYPE_IDS[b_dtype], L.DTYPE_IDS[c_dtype]
    touched = (_extent(m, ldc, n, c_dtype), _extent(m, lda, k, a_dtype), _extent(n, ldb, k, b_dtype))
    if a_dtype in FP8:
        sa, sb = scale_a or None, scale_b or None
        return MatrixProgram(GEMM_FP8, "tgm_gemm_fp8", _tiles(m, n, GEMM_FP8), est,
                             lambda out, x, y, s: (x, adt, lda, m, y, bdt, ldb, n, k, sa, sb, out, cdt, ldc, s),
                             touched)
    if scale_a or scale_b:
        raise ValueError("per-tensor scales apply to FP8 operands only")
    kernel = dense_kernel(m, n, k)
    return MatrixProgram(kernel, "tgm_gemm_dense", _tiles(m, n, kernel), est,
                         lambda out, x, y, s: (x, adt, m, lda, y, bdt, n, ldb, k, out, cdt, ldc, s), touched)


def transpose_program(dtype: str, rows: int, cols: int) -> MatrixProgram:
    """out[cols, rows] = in[rows, cols]^T for 1- or 2-byte elements (slots out, a): the staging
    copy that puts a GEMM operand K-contiguous."""
    size = L.DTYPE_SIZES[dtype]
    if size not in (1, 2):
        raise ValueError(f"no transpose kernel for {dtype}")
    name = "tgm_transpose8" if size == 1 else "tgm_transpose16"
    kernel = MatrixKernel(name, "copy", (64, 64, 1), 256)
    return MatrixProgram(kernel, name, _tiles(rows, cols, kernel), Estimates(0, 2 * rows * cols * size),
                         lambda out, a, b, s: (a, rows, cols, cols, out, rows, s), (rows * cols * size,) * 2)


# ----------------------------------------------------------------------------- plugin-buffer path
@dataclass(frozen=True)
class Matrix:
    """A row-major tensor of ``dtype`` (a dtype name) stored at the start of a plugin buffer."""

    buf: object  # MI355XBuffer
    dtype: str
    shape: tuple[int, ...]

    def __post_init__(self) -> None:
        object.__setattr__(self, "shape", tuple(int(x) for x in self.shape))
        if self.dtype not in L.DTYPE_SIZES:
            raise ValueError(f"dtype {self.dtype} is not supported by the MI355X kernels")
        if any(x < 0 for x in self.shape) or self.buf.size < self.nbytes:
            raise ValueError("buffer is smaller than the declared shape")

    @property
    def nbytes(self) -> int:
        return math.prod(self.shape) * L.DTYPE_SIZES[self.dtype]


@dataclass(frozen=True)
class PackedBuffer:
    """``PackedTensor`` (dx12.py:14-47) over plugin storage: ``data`` holds the LSB-first packed
    bytes, ``scales`` is a Matrix of shape ``shape[:-1] + (ceil(K / block_size),)``."""

    data: object  # MI355XBuffer
    format: str
    shape: tuple[int, ...]
    scales: Matrix | None = None
    block_size: int = 32

    def __post_init__(self) -> None:
        """The reference's checks and messages (dx12.py:32-47), with a device buffer for the
        flat uint8 Tensor."""
        object.__setattr__(self, "shape", tuple(int(x) for x in self.shape))
        if self.format not in FORMATS:
            raise ValueError(f"unknown packed format {self.format!r}")
        if not self.shape or any(x < 0 for x in self.shape):
            raise ValueError("packed shape must contain nonnegative dimensions")
        if not hasattr(self.data, "address") or not hasattr(self.data, "dev"):
            raise ValueError("packed data must be an MI355X device buffer")
        if self.data.size < packed_nbytes(self.format, math.prod(self.shape)):
            raise ValueError("packed storage is smaller than the declared shape")
        if self.block_size < 1:
            raise ValueError("packed block size must be positive")
        if self.scales is not None:
            expected = self.shape[:-1] + (-(-self.shape[-1] // self.block_size),)
            if tuple(self.scales.shape) != expected or self.scales.buf.dev is not self.data.dev:
                raise ValueError("packed scales have incompatible shape or device")

    @property
    def dev(self):
        return self.data.dev

    def desc(self) -> PackedDesc:
        s = self.scales
        return PackedDesc(self.format, self.shape, self.data.size, s.buf.address if s else None,
                          s.dtype if s else None, self.block_size)

    def default_dtype(self) -> str:
        """Unscaled integers decode to int32, unscaled floats to float32, scaled data to at least
        float32 (float64 scales keep float64) -- dx12.py:57-64."""
        if self.scales is not None:
            return "float64" if self.scales.dtype == "float64" else "float32"
        return "int32" if self.format in ("int4", "uint4") else "float32"

    def unpack(self, dtype: str | None = None) -> Matrix:
        return unpack(self, dtype)

    def matmul(self, other: Matrix) -> Matrix:
        """deq(self)[N, K] @ other[K, M] with other given K-last as [M, K] rows (matvec for one row)."""
        return matmul_nt(other, self)


def _dev(x: Matrix | PackedBuffer):
    return x.dev if isinstance(x, PackedBuffer) else x.buf.dev


def _alloc(dev, dtype: str, shape: tuple[int, ...]) -> Matrix:
    nbytes = max(math.prod(shape) * L.DTYPE_SIZES[dtype], 1)
    return Matrix(dev.allocator.alloc(nbytes), dtype, shape)


def unpack(p: PackedBuffer, dtype: str | None = None) -> Matrix:
    """Decode on the device (PackedTensor.unpack, dx12.py:49-106): scales applied at their K-block
    boundaries in float32 (float64 for float64 scales or output), then cast to ``dtype``."""
    dtype = dtype or p.default_dtype()
    out = _alloc(p.dev, dtype, p.shape)
    if math.prod(p.shape):
        unpack_program(p.desc(), dtype)(out.buf, p.data, p.scales.buf if p.scales else None)
    return out


def _check_pair(a_shape: tuple[int, ...], b_shape: tuple[int, ...]) -> None:
    if len(a_shape) != 2 or len(b_shape) != 2 or a_shape[1] != b_shape[1]:
        raise ValueError("matrix operands must have compatible rank-two shapes")


def matmul_nt(a: Matrix | PackedBuffer, b: Matrix | PackedBuffer, dtype: str | None = None) -> Matrix:
    """``a @ b^T`` with both operands K-last (a [M, K], b [N, K]) -> [M, N], fp32 accumulation,
    rounded once to ``dtype`` (default float32, the accumulator of these operand kinds).

    A packed ``b`` with activations ``a`` runs family 1 / 2 (GEMV for M <= 16, else the dequant
    GEMM); two packed FP4 / FP6 operands run the scaled-MFMA GEMM; two bf16 / f16 / FP8 matrices
    run the ordinary MFMA GEMM.  Other combinations raise ``ValueError``: this path has only the
    native kernels (the torch adapter falls back to the exact-width GEMM).
    """
    _check_pair(a.shape, b.shape)
    dtype = dtype or "float32"
    if dtype not in OUTPUTS:
        raise ValueError(f"output dtype {dtype} is not bf16, f16 or f32")
    dev = _dev(b)
    if _dev(a) is not dev:
        raise ValueError("matrix operands must belong to one device")
    m, k = a.shape
    n = b.shape[0]
    out = _alloc(dev, dtype, (m, n))
    if not (m and n):
        return out
    if isinstance(a, PackedBuffer) and isinstance(b, PackedBuffer):
        if a.format not in MX_FORMATS or b.format not in MX_FORMATS:
            raise ValueError("two packed operands need FP4 / FP6 formats")
        if a.format == b.format == "fp6_e3m2":
            # gfx950's scaled MFMA does not sum E3M2 x E3M2 products exactly: A decodes exactly
            # to bf16 and B stays packed in the weight kernels
            x = unpack(a, "bfloat16")
            weight_program(b.desc(), m, "bfloat16", k, dtype, n)(out.buf, b.data, x.buf)
            dev.allocator.free(x.buf, x.buf.size)  # reused only once the product has run
        else:
            mx_program(a.desc(), b.desc(), dtype, n)(out.buf, a.data, b.data)
    elif isinstance(b, PackedBuffer):
        if a.dtype not in ACTIVATIONS:
            raise ValueError(f"activations of dtype {a.dtype} have no packed-weight kernel")
        weight_program(b.desc(), m, a.dtype, k, dtype, n)(out.buf, b.data, a.buf)
    elif isinstance(a, PackedBuffer):
        raise ValueError("a packed left operand takes activations on the right: use matmul_nt(x, W)")
    else:
        ok = (a.dtype in FP8 and b.dtype in FP8) or (a.dtype in ("bfloat16", "float16") and b.dtype == a.dtype)
        if not ok:
            raise ValueError(f"no MFMA GEMM for {a.dtype} x {b.dtype}")
        dense_program(a.dtype, m, k, b.dtype, n, k, k, dtype, n)(out.buf, a.buf, b.buf)
    return out


def matvec(matrix: PackedBuffer, vector: Matrix, output_dtype: str | None = None) -> Matrix:
    """``deq(matrix)[N, K] @ vector[K]`` -> [N] on the GEMV (the reference's matvec with the
    default thread=None, a one-column matmul, linalg.py:226-247)."""
    if len(matrix.shape) != 2 or len(vector.shape) != 1 or matrix.shape[1] != vector.shape[0]:
        raise ValueError("matvec expects a matrix and matching vector on one device")
    y = matmul_nt(Matrix(vector.buf, vector.dtype, (1, vector.shape[0])), matrix, output_dtype)
    return Matrix(y.buf, y.dtype, (matrix.shape[0],))
