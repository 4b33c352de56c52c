"""Scheduled matrix reductions -> the MFMA GEMMs (the reference's ``a @ b`` rewrite on UOps).

alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/matmul.py:51-246 finds the scheduled
kernels that are plain matrix products and replaces each one's CALL with its LinAlg GEMM before
memory planning.  This is that pass over the kernel graphs of ``uop/ops.py``:

* ``match_matmul(sink)`` accepts a kernel that stores one value per (row, column) point of two
  constant ranges, where the value is one ADD-REDUCE over a third (REDUCE-typed) range of the
  product of two INDEXed parameters (each optionally cast to the accumulator), optionally
  followed by a cast or by any elementwise epilogue.  Every index must be affine in the three
  ranges with the strides of a dense matrix: output ``row * n + col``; left ``row * k + i``
  (row-major) or ``i * m + row`` (stored K-major, "transposed"); right ``i * n + col`` (row-major
  [K, N]) or ``col * k + i`` (stored [N, K], "transposed").  Broadcast or data-dependent
  addressing, a second output, aliasing between output and inputs, too-small parameters and
  kernels carrying explicit optimisation options are left alone (matmul.py:51-128).
* ``lower_matmul(linear, input_uops)`` replaces each matched CALL whose operands have a native
  kernel -- bf16 x bf16 or f16 x f16 (``tgm_gemm_dense``, K steps of 64), FP8 x FP8
  (``tgm_gemm_fp8``, K steps of 128), fp32 accumulation -- with: a transpose into a new buffer
  for each operand not already in the GEMM's K-contiguous layout (A [M, K], B [N, K]), or a copy
  for one that is a rebindable input (``input_uops``: its storage may change between replays);
  when K is not a multiple of the step, a rendered copy of each operand into a K-contiguous
  buffer padded with zero columns instead; the product; and, when the kernel has an epilogue,
  the original kernel with the reduction replaced by a read of the product's fp32 result
  (matmul.py:152-232: arbitrary post-matrix expressions stay ordinary kernels).  Everything
  else keeps its CALL.

Products of two bf16 / f16 / FP8 values are exact in fp32 on these GEMMs and their sums are
fp32; a kernel that rounds the product to the operand dtype before the cast (``(a * b).cast``)
is run with the matrix unit's own (exact) products, as the reference lets LinAlg own its
arithmetic (matmul.py:58-60).
"""

from __future__ import annotations

from dataclasses import dataclass
from itertools import permutations

from tinygrad_mi355x.codegen import program as P
from tinygrad_mi355x.uop.ops import FP8_DTYPES, AxisType, DType, KernelInfo, Ops, UOp, dtypes

MATRIX_DTYPES = (dtypes.float16, dtypes.bfloat16, dtypes.float32, *FP8_DTYPES)
OUTPUT_DTYPES = (dtypes.float16, dtypes.bfloat16, dtypes.float32)


@dataclass(frozen=True)
class MatmulSpec:
    """A matched product: sizes, the output / left / right PARAMs, the reduction and its
    accumulator dtype, the output index, whether an epilogue follows, and the operand layouts
    (``transposed[0]``: left stored [K, M]; ``transposed[1]``: right stored [N, K])."""

    m: int
    n: int
    k: int
    output: UOp
    left: UOp
    right: UOp
    accumulator: DType
    reduction: UOp
    output_index: UOp
    epilogue: bool
    transposed: tuple[bool, bool] = (False, False)


def _affine(value: UOp, axes: tuple[UOp, ...]) -> tuple[int, ...] | None:
    """``value`` as (constant, coefficient of each axis), or None when it is not affine with
    constant integer coefficients."""
    if value in axes:
        return (0, *(int(value is a) for a in axes))
    if value.op is Ops.CONST and isinstance(value.arg, int) and not isinstance(value.arg, bool):
        return (value.arg, *(0,) * len(axes))
    if value.op not in (Ops.ADD, Ops.SUB, Ops.MUL) or len(value.src) != 2:
        return None
    a, b = (_affine(s, axes) for s in value.src)
    if a is None or b is None:
        return None
    if value.op is Ops.ADD:
        return tuple(x + y for x, y in zip(a, b))
    if value.op is Ops.SUB:
        return tuple(x - y for x, y in zip(a, b))
    if not any(a[1:]):
        return tuple(a[0] * y for y in b)
    if not any(b[1:]):
        return tuple(b[0] * x for x in a)
    return None  # a product of two axes


def _strip_cast(x: UOp, dt: DType) -> UOp:
    return x.src[0] if x.op is Ops.CAST and x.dtype == dt else x


def match_matmul(sink: UOp) -> MatmulSpec | None:
    """The matrix product a scheduled kernel computes, or None (see the module docstring)."""
    if sink.op is not Ops.SINK or len(sink.src) != 1 or not isinstance(sink.arg, KernelInfo):
        return None
    if sink.arg.applied_opts or sink.arg.opts_to_apply is not None:
        return None
    end = sink.src[0]
    if end.op is not Ops.END or len(end.src) != 3:
        return None
    store = end.src[0]
    if store.op is not Ops.STORE or len(store.src) != 2:
        return None
    target, value = store.src
    if target.op is not Ops.INDEX or len(target.src) != 2 or target.src[0].op is not Ops.PARAM:
        return None
    reduces = [u for u in value.toposort() if u.op is Ops.REDUCE]
    if len(reduces) != 1:
        return None
    red = reduces[0]
    if red.arg is not Ops.ADD or len(red.src) != 2:
        return None
    epilogue = value is not red and not (value.op is Ops.CAST and value.src[0] is red)
    acc = red.dtype
    product, axis_k = _strip_cast(red.src[0], acc), red.src[1]
    if product.op is not Ops.MUL or len(product.src) != 2:
        return None
    inputs = tuple(_strip_cast(s, acc) for s in product.src)
    if any(x.op is not Ops.INDEX or len(x.src) != 2 or x.src[0].op is not Ops.PARAM or x.dtype not in MATRIX_DTYPES
           for x in inputs):
        return None
    axes = (*end.src[1:], axis_k)
    if len(set(axes)) != 3 or any(a.op is not Ops.RANGE or a.src[0].op is not Ops.CONST or
                                  not isinstance(a.src[0].arg, int) or a.src[0].arg <= 0 for a in axes):
        return None
    if axis_k.arg[-1] is not AxisType.REDUCE:
        return None
    for row, col in permutations(end.src[1:]):
        m, n, k = (a.src[0].arg for a in (row, col, axis_k))
        order = (row, col, axis_k)
        if _affine(target.src[1], order) != (0, n, 1, 0):
            continue
        for left, right in permutations(inputs):
            li, ri = _affine(left.src[1], order), _affine(right.src[1], order)
            if li not in ((0, k, 0, 1), (0, 1, 0, m)) or ri not in ((0, 0, 1, n), (0, 0, k, 1)):
                continue
            params = (target.src[0], left.src[0], right.src[0])
            if params[0] in params[1:] or any(p.max_numel() < size for p, size in zip(params, (m * n, m * k, k * n))):
                continue
            return MatmulSpec(m, n, k, *params, acc, red, target.src[1], epilogue,
                              (li == (0, 1, 0, m), ri == (0, 0, k, 1)))
    return None


def native_kernel(spec: MatmulSpec) -> str | None:
    """``"dense"`` / ``"fp8"`` when a native GEMM takes this product, else None."""
    a, b = spec.left.dtype, spec.right.dtype
    if spec.accumulator != dtypes.float32:
        return None
    if not spec.epilogue and spec.output.dtype not in OUTPUT_DTYPES:
        return None
    if a == b and a in (dtypes.bfloat16, dtypes.float16):
        return "dense"
    if a in FP8_DTYPES and b in FP8_DTYPES:
        return "fp8"
    return None


def _k_step(kind: str) -> int:
    return 64 if kind == "dense" else 128  # the GEMMs' K step (tgm_gemm_dense / tgm_gemm_fp8)


def _storage(dt: DType) -> DType:
    """Copies move FP8 elements as their bytes (the renderer decodes FP8 loads but does not encode)."""
    return dtypes.uint8 if dt in FP8_DTYPES else dt


def _program(p) -> UOp:
    return UOp(Ops.PROGRAM, None, (), p)


def _copy_call(device, arg: UOp, dt: DType, size: int) -> tuple[UOp, UOp]:
    """A rendered element copy of ``arg`` into a new buffer (the reference's staging kernel,
    matmul.py:218-226): (call, new buffer)."""
    staged = UOp.new_buffer(device, size, dt)
    sdt = _storage(dt)
    dest, src = UOp.param(0, sdt, size, device), UOp.param(1, sdt, size, device)
    axis = UOp.range(size, 0)
    sink = dest.index(axis).store(src.index(axis)).end(axis).sink(arg=KernelInfo(name="mi355x_matrix_input"))
    return UOp.call(sink, staged, arg), staged


def _pad_call(device, arg: UOp, dt: DType, rows: int, k: int, kp: int, k_major: bool) -> tuple[UOp, UOp]:
    """A rendered copy of an operand into a new K-contiguous [rows, kp] buffer, zero past column k
    (the reference's tail padding, codegen/linalg.py:61-87): ``arg`` holds [rows, k] or, K-major,
    [k, rows].  Zero columns add nothing to the product.  (call, new buffer)."""
    staged = UOp.new_buffer(device, rows * kp, dt)
    sdt = _storage(dt)
    dest, src = UOp.param(0, sdt, rows * kp, device), UOp.param(1, sdt, rows * k, device)
    r, c = UOp.range(rows, 0), UOp.range(kp, 1)
    value = src.index(c * rows + r if k_major else r * k + c, c < k)  # gated: no read past column k
    ranges = (c, r) if k_major else (r, c)  # the source's contiguous axis varies fastest
    sink = dest.index(r * kp + c).store(value).end(*ranges).sink(arg=KernelInfo(name="mi355x_matrix_pad"))
    return UOp.call(sink, staged, arg), staged


def _lower_call(call: UOp, inputs: set) -> tuple[UOp, ...]:
    if call.op is not Ops.CALL or call.src[0].op is not Ops.SINK:
        return (call,)
    spec = match_matmul(call.src[0])
    kind = native_kernel(spec) if spec is not None else None
    if kind is None:
        return (call,)
    slots = (spec.output.arg.slot, spec.left.arg.slot, spec.right.arg.slot)
    if any(s + 1 >= len(call.src) for s in slots):
        return (call,)
    output, left, right = (call.src[s + 1] for s in slots)
    for arg, param in ((output, spec.output), (left, spec.left), (right, spec.right)):
        # the GEMM reads and writes whole matrices: an argument that does not hold its
        # parameter keeps the ordinary kernel, whose launch rejects it
        if arg.op is not Ops.BUFFER or arg.dtype != param.dtype or arg.max_numel() < param.max_numel():
            return (call,)
    if output is left or output is right:
        return (call,)  # the call writes the product over an operand
    if not spec.epilogue and output in inputs:
        return (call,)  # a rebindable output cannot be checked for the GEMM's alignment here
    device = spec.output.arg.device
    m, n, k = spec.m, spec.n, spec.k
    a_dt, b_dt = spec.left.dtype, spec.right.dtype
    calls: list[UOp] = []
    kp = -(-k // _k_step(kind)) * _k_step(kind)
    if kp != k:  # K padded with zero columns to the GEMM's step, both operands K-contiguous
        pad_a, a_buf = _pad_call(device, left, a_dt, m, k, kp, spec.transposed[0])
        pad_b, b_buf = _pad_call(device, right, b_dt, n, k, kp, not spec.transposed[1])
        calls += [pad_a, pad_b]
    else:
        # A as [M, K] rows, B as [N, K] rows, in fresh buffers where the layout or a
        # rebindable input requires it
        if spec.transposed[0]:
            a_buf = UOp.new_buffer(device, m * k, a_dt)
            calls.append(UOp.call(_program(P.transpose_program(a_dt.name, k, m)), a_buf, left))
        elif left in inputs:
            copy, a_buf = _copy_call(device, left, a_dt, m * k)
            calls.append(copy)
        else:
            a_buf = left
        if not spec.transposed[1]:
            b_buf = UOp.new_buffer(device, n * k, b_dt)
            calls.append(UOp.call(_program(P.transpose_program(b_dt.name, k, n)), b_buf, right))
        elif right in inputs:
            copy, b_buf = _copy_call(device, right, b_dt, n * k)
            calls.append(copy)
        else:
            b_buf = right
    out_dt = dtypes.float32 if spec.epilogue else spec.output.dtype
    target = UOp.new_buffer(device, m * n, out_dt) if spec.epilogue else output
    gemm = P.dense_program(a_dt.name, m, kp, b_dt.name, n, kp, kp, out_dt.name, n)
    calls.append(UOp.call(_program(gemm), target, a_buf, b_buf))
    if spec.epilogue:
        tmp = UOp.param(len(call.src) - 1, dtypes.float32, m * n, device)
        body = call.src[0].substitute({spec.reduction: tmp.index(spec.output_index)})
        calls.append(UOp.call(body, *call.src[1:], target))
    return tuple(calls)


def lower_matmul(linear: UOp, input_uops: tuple[UOp, ...] = ()) -> UOp:
    """``linear`` with every matched product CALL replaced by its native GEMM calls."""
    if linear.op is not Ops.LINEAR:
        raise ValueError("lower_matmul takes a LINEAR of CALLs")
    inputs = set(input_uops)
    return UOp.linear(*(c for call in linear.src for c in _lower_call(call, inputs)))
