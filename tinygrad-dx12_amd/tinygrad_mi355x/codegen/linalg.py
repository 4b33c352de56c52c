"""Explicit matrix API over packed and ordinary tensors on the MI355X device.

Mirrors ``matmul``/``matvec`` of alexandreteles/tinygrad-dx12
(src/tinygrad_dx12/codegen/linalg.py:136-298): the same signatures, validation,
intermediate and accumulator dtypes, scope names and "auto falls back, explicit
scopes raise" behaviour.  What changes is what runs:

* a packed K-blocked weight times activations goes to kernel family 1 (fused
  dequant GEMV, M <= 16) or family 2 (dequant-to-bf16 MFMA GEMM);
* two packed FP4 / FP6 operands (``matmul_nt``), each E8M0 block-32 scaled or unscaled, go to
  the scaled-MFMA GEMM (E3M2 x E3M2, which that MFMA does not sum exactly, decodes A to bf16
  for the weight GEMM);
* two ordinary bf16 or f16 operands go to the ordinary MFMA GEMM (``tgm_gemm_dense``), two
  FP8 operands to the same GEMM with the FP8 values decoded to bf16 (``tgm_gemm_fp8``);
* everything else runs the exact-width device GEMM ``tgm_gemm_plain`` -- the
  analogue of the reference's ordinary-matmul fallback.

Every path is a gfx950 kernel; CPU tensors are rejected.

``matmul_nt(a, b)`` is an extension: ``a @ b.T`` with both operands stored K-last.
The reference has no such entry point, so a K-blocked packed right operand cannot
express ``A @ W.T`` there (its ``b.shape[0] == K`` check, linalg.py:166).
"""

from __future__ import annotations

import os
import warnings

import torch

from tinygrad_mi355x import dtype as D
from tinygrad_mi355x.codegen import program as P
from tinygrad_mi355x.codegen.decomp.mi355x import MX_FORMATS, PackedTensor, matrix_intermediate
from tinygrad_mi355x.renderer.linalg import (ACTIVATION_DTYPES, DENSE_DTYPES, FP8_DTYPES, GEMM_DENSE, GEMM_FP8,
                                             GEMM_MX, GEMM_MX_GENERAL, GEMM_W, GEMV, GEMV_MAX_ROWS, OUTPUT_DTYPES,
                                             WEIGHT_SCALE_DTYPES, MatrixKernel, _accumulator, mx_kernel)
from tinygrad_mi355x.runtime import kernels as K

SCOPES = ("auto", "Wave", "ThreadGroup", "tiled")
# Automatic matrix lowering switch (the reference's DX12_LINALG ContextVar, linalg.py:15).
MI355X_LINALG = int(os.environ.get("MI355X_LINALG", "1"))
# Rejections cached per exact candidate, like renderer.matrix_failures (linalg.py:216-220).
matrix_failures: dict[tuple, str] = {}

_ACC_IDS = {torch.float32: 13, torch.float64: 14, torch.int32: 5, torch.uint32: 6, torch.int64: 7, torch.uint64: 8}


def _name(dt: torch.dtype) -> str:
    """A torch dtype's name in the kernel programs (ValueError for dtypes the kernels lack)."""
    K.dtype_id(dt)
    return str(dt).rsplit(".", 1)[-1]


def _device(x: torch.Tensor | PackedTensor) -> torch.device:
    return x.data.device if isinstance(x, PackedTensor) else x.device


def _plain_acc(out_dtype: torch.dtype) -> torch.dtype:
    acc = D.sum_acc_dtype(out_dtype)
    return acc if acc in _ACC_IDS else torch.float32


def plain_matmul(lhs: torch.Tensor, rhs: torch.Tensor, out_dtype: torch.dtype, acc_dtype: torch.dtype | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Exact-width device GEMM ``lhs @ rhs`` (products and sums at ``acc_dtype``).

    ``lhs`` [M,K] and ``rhs`` [K,N] may be any strided views; the result is [M,N].
    """
    K.require_device(lhs)
    m, k = lhs.shape
    n = rhs.shape[1]
    acc = acc_dtype or _plain_acc(out_dtype)
    if acc not in _ACC_IDS:
        acc = _plain_acc(acc)
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=lhs.device)
    if k == 0:
        out.zero_()
        return out
    K.call("tgm_gemm_plain", lhs.data_ptr(), K.dtype_id(lhs.dtype), lhs.stride(0), lhs.stride(1),
           rhs.data_ptr(), K.dtype_id(rhs.dtype), rhs.stride(0), rhs.stride(1),
           out.data_ptr(), K.dtype_id(out_dtype), out.stride(0), out.stride(1), m, n, k, _ACC_IDS[acc],
           K.stream_of(lhs))
    return out


def transpose16(x: torch.Tensor) -> torch.Tensor:
    """Contiguous transpose of a 2-D 16-bit (or, for FP8, 8-bit) tensor on the device (the
    staging copy of a row-major right operand for the NT GEMM)."""
    K.require_device(x)
    rows, cols = x.shape
    out = torch.empty((cols, rows), dtype=x.dtype, device=x.device)
    # the kernel reads row i at x + i * ld_in with unit column stride: any other column
    # stride (a single-row view included) is staged first
    if x.stride(1) != 1 and cols > 1:
        x = x.contiguous()
    name = "tgm_transpose8" if x.element_size() == 1 else "tgm_transpose16"
    K.call(name, x.data_ptr(), rows, cols, x.stride(0) if rows > 1 else cols, out.data_ptr(), rows, K.stream_of(x))
    return out


def _k_rows(x: torch.Tensor) -> torch.Tensor:
    """``x`` with contiguous rows (unit stride along the last axis)."""
    return x if x.stride(1) == 1 or x.shape[1] == 1 else x.contiguous()


def _rows_aligned(x: torch.Tensor) -> bool:
    return x.data_ptr() % 16 == 0 and (x.shape[0] <= 1 or x.stride(0) * x.element_size() % 16 == 0)


def _padded_k(x: torch.Tensor, kp: int) -> torch.Tensor:
    """``x`` [rows, K] as a contiguous [rows, kp] copy with zeros past column K: zero columns on
    both operands add nothing to any product, so the GEMM's K step and 16-byte row alignment
    hold for every K (the staging the UOp rewrite does, codegen/uop_matmul.py)."""
    out = torch.zeros((x.shape[0], kp), dtype=x.dtype, device=x.device)
    out[:, :x.shape[1]].copy_(x)
    return out


def dense_matmul_nt(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype, scale_a: torch.Tensor | None = None,
                    scale_b: torch.Tensor | None = None) -> torch.Tensor:
    """C[M, N] = a[M, K] @ b[N, K]^T on the ordinary MFMA GEMM (bf16 or f16 operands; FP8
    operands decoded exactly to bf16 in registers); ``scale_a`` / ``scale_b`` are optional fp32
    device scalars (FP8 only) that multiply the fp32 sums before rounding.  A K off the GEMM's
    step (64; 128 for FP8) or rows off 16-byte alignment are staged zero-padded."""
    for s in (scale_a, scale_b):
        if s is not None and (s.dtype is not torch.float32 or s.numel() != 1 or s.device != a.device):
            raise ValueError("scales must be single fp32 values on the operands' device")
    a, b = _k_rows(a), _k_rows(b)
    step = (GEMM_FP8 if a.dtype in FP8_DTYPES else GEMM_DENSE).tile[2]
    k0 = a.shape[1]
    if k0 and (k0 % step or not _rows_aligned(a) or not _rows_aligned(b)):
        kp = -(-k0 // step) * step
        a, b = _padded_k(a, kp), _padded_k(b, kp)
    m, k = a.shape
    n = b.shape[0]
    c = torch.empty((m, n), dtype=out_dtype, device=a.device)
    lda, ldb = a.stride(0) if m > 1 else k, b.stride(0) if n > 1 else k
    program = P.dense_program(_name(a.dtype), m, lda, _name(b.dtype), n, ldb, k, _name(out_dtype), n,
                              K.ptr(scale_a) or 0, K.ptr(scale_b) or 0)
    program.launch(c.data_ptr(), a.data_ptr(), b.data_ptr(), K.stream_of(a))
    return c


def _dense_kernel(a: torch.Tensor, b: torch.Tensor, out_dtype: torch.dtype, tile, scope: str) -> MatrixKernel | None:
    if scope == "tiled" or not MI355X_LINALG or out_dtype not in OUTPUT_DTYPES:
        return None
    if a.dtype in FP8_DTYPES and b.dtype in FP8_DTYPES:
        kernel = GEMM_FP8
    elif a.dtype in DENSE_DTYPES and b.dtype is a.dtype:
        kernel = GEMM_DENSE
    else:
        return None
    return kernel if tile is None or tuple(tile) == kernel.tile else None


def _decoded(x: torch.Tensor | PackedTensor, intermediate: torch.dtype) -> torch.Tensor:
    return x.unpack(intermediate) if isinstance(x, PackedTensor) else x


def choose_matrix(weight: PackedTensor | None, activation: torch.Tensor | PackedTensor | None, intermediate: torch.dtype,
                  out_dtype: torch.dtype, m: int, tile: tuple[int, int, int] | None = None,
                  scope: str = "auto") -> MatrixKernel | None:
    """Static gfx950 kernel selection (replaces the LinAlg query of linalg.py:90-133).

    ``weight`` is the K-blocked packed operand ([N, K]), ``activation`` the other operand
    seen as [M, K] (``m`` rows).  Returns the kernel family or ``None`` for ordinary compute.
    """
    if scope == "tiled" or not MI355X_LINALG or weight is None or len(weight.shape) != 2:
        return None
    if out_dtype not in OUTPUT_DTYPES:
        return None
    if isinstance(activation, PackedTensor):
        # two FP4 / FP6 operands, each E8M0 block-32 scaled or unscaled (the FP8 intermediate of
        # two unscaled codes, or fp32 when either is scaled): the scaled MFMA multiplies exactly
        # the decoded values
        def mx_operand(t: PackedTensor) -> bool:
            return t.format in MX_FORMATS and (t.scales is None or (
                t.block_size == 32 and t.scales.dtype is torch.float8_e8m0fnu))

        kernel = None
        if mx_operand(weight) and mx_operand(activation):
            kernel = mx_kernel(activation.format, activation.scales is not None, weight.format,
                               weight.scales is not None, weight.shape[1])
    elif intermediate not in (torch.float16, torch.bfloat16, torch.float32):
        return None
    else:
        if activation is None or activation.dtype not in ACTIVATION_DTYPES:
            return None
        if weight.scales is not None and weight.scales.dtype not in WEIGHT_SCALE_DTYPES:
            return None
        kernel = GEMV if m <= GEMV_MAX_ROWS else GEMM_W
    if kernel is not None and tile is not None and tuple(tile) != kernel.tile:
        return None
    return kernel


def _weight_left(kernel: MatrixKernel, w: PackedTensor, x: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """Y[M, N] = X[M, K] @ deq(W)[N, K]^T through family 1 or 2."""
    n, k = w.shape
    m = x.shape[0]
    if x.stride(1) != 1 and k > 1:
        x = x.contiguous()
    data = w.data if w.data.is_contiguous() else w.data.contiguous()
    scales = w.scales
    if scales is not None and not scales.is_contiguous():
        scales = scales.contiguous()
    y = torch.empty((m, n), dtype=out_dtype, device=x.device)
    ldx = x.stride(0) if m > 1 else k
    program = P.weight_program(w.desc(data, scales), m, _name(x.dtype), ldx, _name(out_dtype), n)
    if program.kernel is not kernel:
        raise K.UnsupportedKernel(f"{kernel.name}: {m} activation rows belong to {program.kernel.name}")
    program.launch(y.data_ptr(), data.data_ptr(), x.data_ptr(), K.stream_of(x))
    return y


def _mx_nt(a: PackedTensor, b: PackedTensor, out_dtype: torch.dtype) -> torch.Tensor:
    """C[M, N] = deq(A)[M, K] @ deq(B)[N, K]^T on the block-scaled MFMA kernel."""
    m, k = a.shape
    n = b.shape[0]
    c = torch.empty((m, n), dtype=out_dtype, device=a.device)
    ad, bd = (t.data if t.data.is_contiguous() else t.data.contiguous() for t in (a, b))
    sa, sb = (None if t.scales is None else t.scales.contiguous() for t in (a, b))
    program = P.mx_program(a.desc(ad, sa), b.desc(bd, sb), _name(out_dtype), n)
    program.launch(c.data_ptr(), ad.data_ptr(), bd.data_ptr(), K.stream_of(ad))
    return c


class MatrixFallbackWarning(UserWarning):
    """A product of packed operands, or one a native kernel rejected, ran on the exact-width
    device GEMM ``tgm_gemm_plain`` (decoded operands, scalar products) instead of a native
    MFMA / GEMV kernel: correct, and much slower."""


# Automatic fallbacks to the exact-width GEMM: operand key -> reason (each warned once).
fallbacks: dict[tuple, str] = {}


def _fall_back(generic, key: tuple, reason: str, warn: bool):
    if key not in fallbacks:
        fallbacks[key] = reason
        if warn:
            warnings.warn(f"MI355X matrix product on tgm_gemm_plain ({reason}); operands {key[1:]}",
                          MatrixFallbackWarning, stacklevel=4)
    return generic()


def _dispatch(native, generic, kernel: MatrixKernel | None, scope: str, key: tuple, packed: bool = False):
    """Run ``native`` when a kernel was chosen; auto falls back, explicit scopes raise
    (linalg.py:193-223).  An automatic fallback is recorded in ``fallbacks`` and, for packed
    operands or a native rejection, warned once per operand key (``MatrixFallbackWarning``)."""
    automatic = scope == "auto"
    if kernel is None:
        if scope == "tiled":
            return generic()
        if automatic:
            return _fall_back(generic, key, "no native kernel for this operand combination", packed)
        raise RuntimeError(f"MI355X {scope} candidate rejected: no native kernel for this operand combination")
    if key in matrix_failures:
        if automatic:
            return _fall_back(generic, key, matrix_failures[key], True)
        raise RuntimeError(f"MI355X {scope} candidate rejected: {matrix_failures[key]}")
    try:
        return native()
    except (K.UnsupportedKernel, ValueError) as error:
        matrix_failures[key] = str(error)
        if automatic:
            return _fall_back(generic, key, str(error), True)
        raise RuntimeError(f"MI355X {scope} candidate rejected: {error}") from error


def _key(kernel, *operands, out_dtype, m) -> tuple:
    parts = []
    for x in operands:
        if isinstance(x, PackedTensor):
            parts.append((x.format, x.shape, None if x.scales is None else x.scales.dtype, x.block_size,
                          x.data.data_ptr() % 16))
        else:
            parts.append((x.dtype, tuple(x.shape), tuple(x.stride()), x.data_ptr() % 16))
    return (kernel.name if kernel else None, m, out_dtype, *parts)


def _require(*operands) -> None:
    for x in operands:
        K.require_device(x.data if isinstance(x, PackedTensor) else x)


def _validate(a, b, scope: str, tile) -> torch.device:
    if scope not in SCOPES:
        raise ValueError(f"unknown matrix scope {scope!r}")
    device = _device(a)
    if device != _device(b):
        raise ValueError("matrix operands must belong to one device")
    if tile is not None and any(x < 1 for x in tile):
        raise ValueError("matrix tile dimensions must be positive")
    return device


def _empty_result(m: int, n: int, k: int, out_dtype: torch.dtype, device) -> torch.Tensor:
    return torch.zeros((m, n), dtype=out_dtype, device=device) if k == 0 else torch.empty((m, n), dtype=out_dtype, device=device)


def matmul(a: torch.Tensor | PackedTensor, b: torch.Tensor | PackedTensor, scope: str = "auto",
           tile: tuple[int, int, int] | None = None, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Multiply two matrices on the MI355X device (linalg.py:136-223).

    ``scope`` is ``auto`` (native kernel when one exists, exact ordinary compute
    otherwise), ``Wave``/``ThreadGroup`` (a native kernel is required; otherwise
    ``RuntimeError("... candidate rejected ...")``) or ``tiled`` (ordinary compute).
    ``dtype`` declares the output precision; native kernels accumulate in fp32 and
    round once.  A packed ``a`` of logical shape [N, K] times ``b`` [K, M] runs the
    fused-dequant kernels; the [N, M] result is returned as a transposed view.
    """
    device = _validate(a, b, scope, tile)
    if len(a.shape) != 2 or len(b.shape) != 2 or a.shape[1] != b.shape[0]:
        raise ValueError("matrix operands must have compatible rank-two shapes")
    intermediate = matrix_intermediate(a, b)
    packed = isinstance(a, PackedTensor) or isinstance(b, PackedTensor)
    lhs_dt = intermediate if packed else a.dtype
    rhs_dt = intermediate if packed else b.dtype
    out_dtype = dtype or _accumulator(lhs_dt, rhs_dt)
    m, k = a.shape
    n = b.shape[1]
    if 0 in (m, n, k):
        return _empty_result(m, n, k, out_dtype, device)
    _require(a, b)

    def generic() -> torch.Tensor:
        return plain_matmul(_decoded(a, intermediate), _decoded(b, intermediate), out_dtype)

    if isinstance(a, PackedTensor) and isinstance(b, torch.Tensor):
        kernel = choose_matrix(a, b, intermediate, out_dtype, n, tile, scope)
        key = _key(kernel, a, b, out_dtype=out_dtype, m=n)
        return _dispatch(lambda: _weight_left(kernel, a, b.t(), out_dtype).t(), generic, kernel, scope, key, True)
    if not packed:
        kernel = _dense_kernel(a, b, out_dtype, tile, scope)
        key = _key(kernel, a, b, out_dtype=out_dtype, m=m)
        # b [K, N]: a transposed view of a K-last tensor binds directly, a row-major one is staged
        native = lambda: dense_matmul_nt(a, b.t() if b.stride(0) == 1 else transpose16(b), out_dtype)  # noqa: E731
        return _dispatch(native, generic, kernel, scope, key)
    return _dispatch(None, generic, None, scope, _key(None, a, b, out_dtype=out_dtype, m=m), True)


def matmul_nt(a: torch.Tensor | PackedTensor, b: torch.Tensor | PackedTensor, scope: str = "auto",
              tile: tuple[int, int, int] | None = None, dtype: torch.dtype | None = None) -> torch.Tensor:
    """``a @ b.T`` with both operands stored K-last: a [M, K], b [N, K] -> [M, N].

    Dtype rules are those of ``matmul(a, b.T)``.  Two packed FP4 / FP6 operands (E8M0
    block-32 scales or none) run the scaled-MFMA GEMM; one packed operand runs the
    fused-dequant families; bf16 / f16 / FP8 pairs run the ordinary MFMA GEMM; anything else
    runs ordinary exact compute.
    """
    device = _validate(a, b, scope, tile)
    if len(a.shape) != 2 or len(b.shape) != 2 or a.shape[1] != b.shape[1]:
        raise ValueError("matrix operands must have compatible rank-two shapes")
    intermediate = matrix_intermediate(a, b)
    packed = isinstance(a, PackedTensor) or isinstance(b, PackedTensor)
    lhs_dt = intermediate if packed else a.dtype
    rhs_dt = intermediate if packed else b.dtype
    out_dtype = dtype or _accumulator(lhs_dt, rhs_dt)
    m, k = a.shape
    n = b.shape[0]
    if 0 in (m, n, k):
        return _empty_result(m, n, k, out_dtype, device)
    _require(a, b)

    def generic() -> torch.Tensor:
        return plain_matmul(_decoded(a, intermediate), _decoded(b, intermediate).t(), out_dtype)

    if isinstance(a, PackedTensor) and isinstance(b, PackedTensor):
        kernel = choose_matrix(b, a, intermediate, out_dtype, m, tile, scope)
        key = _key(kernel, a, b, out_dtype=out_dtype, m=m)
        if kernel in (GEMM_MX, GEMM_MX_GENERAL) and a.format == b.format == "fp6_e3m2":
            # gfx950's scaled MFMA does not sum E3M2 x E3M2 products exactly; A decodes exactly to
            # bf16 and B stays packed in the weight GEMM (or GEMV for a few rows of A)
            family = GEMV if m <= GEMV_MAX_ROWS else GEMM_W
            native = lambda: _weight_left(family, b, a.unpack(torch.bfloat16), out_dtype)  # noqa: E731
        else:
            native = lambda: _mx_nt(a, b, out_dtype)  # noqa: E731
        return _dispatch(native, generic, kernel, scope, key, True)
    if isinstance(b, PackedTensor):
        kernel = choose_matrix(b, a, intermediate, out_dtype, m, tile, scope)
        key = _key(kernel, b, a, out_dtype=out_dtype, m=m)
        return _dispatch(lambda: _weight_left(kernel, b, a, out_dtype), generic, kernel, scope, key, True)
    if isinstance(a, PackedTensor):
        kernel = choose_matrix(a, b, intermediate, out_dtype, n, tile, scope)
        key = _key(kernel, a, b, out_dtype=out_dtype, m=n)
        return _dispatch(lambda: _weight_left(kernel, a, b, out_dtype).t(), generic, kernel, scope, key, True)
    kernel = _dense_kernel(a, b, out_dtype, tile, scope)
    key = _key(kernel, a, b, out_dtype=out_dtype, m=m)
    return _dispatch(lambda: dense_matmul_nt(a, b, out_dtype), generic, kernel, scope, key)


def linear(x: torch.Tensor, weight: PackedTensor | torch.Tensor, dtype: torch.dtype | None = None) -> torch.Tensor:
    """``x @ weight.T`` for activations x [..., K] and a K-last weight [N, K] (extension)."""
    lead = tuple(x.shape[:-1])
    flat = x.reshape(-1, x.shape[-1])
    out = matmul_nt(flat, weight, dtype=dtype)
    return out.reshape(*lead, out.shape[-1])


def matvec(matrix: torch.Tensor | PackedTensor, vector: torch.Tensor, output_dtype: torch.dtype | None = None,
           thread: bool | None = None) -> torch.Tensor:
    """Matrix-vector product through the shared matrix path (linalg.py:226-298).

    ``thread=None`` is a one-column ``matmul``; ``thread=False`` selects ordinary exact
    compute; ``thread=True`` asks for the native GEMV and silently falls back when the
    operands have none, as the reference's thread scope does.
    """
    device = _device(matrix)
    if len(matrix.shape) != 2 or vector.dim() != 1 or matrix.shape[1] != vector.shape[0] or device != vector.device:
        raise ValueError("matvec expects a matrix and matching vector on one device")
    intermediate = matrix_intermediate(matrix, vector)
    output_dtype = output_dtype or _accumulator(intermediate, intermediate)
    if thread is None:
        return matmul(matrix, vector.reshape(-1, 1), dtype=output_dtype).reshape(matrix.shape[0])
    n, k = matrix.shape
    if not n or not k:
        return _empty_result(n, 1, k, output_dtype, device).reshape(n)
    _require(matrix, vector)

    def generic() -> torch.Tensor:
        return plain_matmul(_decoded(matrix, intermediate), vector.reshape(-1, 1), output_dtype).reshape(n)

    if thread is False or not isinstance(matrix, PackedTensor):
        return generic()
    kernel = choose_matrix(matrix, vector.reshape(1, -1), intermediate, output_dtype, 1, None, "auto")
    if kernel is not GEMV:
        return generic()
    key = _key(kernel, matrix, vector, out_dtype=output_dtype, m=1)
    return _dispatch(lambda: _weight_left(kernel, matrix, vector.reshape(1, -1), output_dtype).reshape(n),
                     generic, kernel, "auto", key)
