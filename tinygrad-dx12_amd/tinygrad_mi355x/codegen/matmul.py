"""Rewrite the matrix products of a traced program onto the MI355X GEMM family.

The reference recognises scheduled rank-two matrix reductions in tinygrad's kernel graph and
lowers them to its native LinAlg GEMM before scalar expansion, keeping autograd and JIT replay
working (alexandreteles/tinygrad-dx12 src/tinygrad_dx12/codegen/matmul.py:13-246).  tinygrad is
not installed here; the graph a caller hands over here is a ``torch.fx`` GraphModule, and
the rewrite works on its nodes with the same conservative rules:

* only a product of two rank-two operands with static shapes is a candidate (``match_matmul``);
  batched or broadcast products, operands of other dtypes and nodes a caller pinned (the
  ``tgm_keep`` meta flag, the analogue of a kernel carrying explicit optimizer options,
  matmul.py:61-62) keep their ordinary lowering;
* transposes feeding the product are absorbed into the operand layout (matmul.py:120-131);
* a product whose only use is an elementwise epilogue is still rewritten; the epilogue stays an
  ordinary node after the native product (matmul.py:240-245);
* a right operand that is ``unpack(packed)`` -- the decode of a PackedTensor -- feeds the
  packed-weight kernels directly (family 1 GEMV / family 2 GEMM), so the decoded weight is never
  materialised;
* an FP8 product -- torch's ``torch._scaled_mm(a, b, scale_a, scale_b, out_dtype=...)`` with
  per-tensor fp32 scales, a [M, K] row-major and b [K, N] column-major (the layout it requires)
  -- runs the FP8 GEMM (``tgm_gemm_fp8``: FP8 values decoded exactly to bf16, fp32 sums times
  scale_a * scale_b, rounded once to out_dtype), as the reference's rewrite hands FP8 operands
  to its LinAlg GEMM (matmul.py:51-128 with renderer/linalg.py:12-13);
* operands whose rows are not 16-byte aligned are staged by a copy at run time (the
  reference's ``dx12_matrix_input`` staging, matmul.py:218-226).

The replacement keeps autograd: ``native_matmul`` is an autograd Function whose backward
products run on the same kernels (and on the exact-width device GEMM where a shape has no
MFMA tiling).  Nothing here computes on the CPU.
"""

from __future__ import annotations

import operator
from dataclasses import dataclass

import torch
import torch.fx
import torch.nn.functional as F
from torch.fx.passes.shape_prop import ShapeProp

from tinygrad_mi355x.codegen import linalg
from tinygrad_mi355x.codegen.decomp.mi355x import PackedTensor, unpack
from tinygrad_mi355x.renderer.linalg import DENSE_DTYPES, FP8_DTYPES, OUTPUT_DTYPES
from tinygrad_mi355x.runtime import kernels as K

MATMUL_FUNCTIONS = (torch.matmul, torch.mm, operator.matmul)
MATMUL_METHODS = ("matmul", "mm", "__matmul__")
SCALED_MM = getattr(torch, "_scaled_mm", None)  # torch's FP8 matrix product
KEEP = "tgm_keep"
ELEMENTWISE = (torch.relu, F.relu, F.gelu, F.silu, torch.sigmoid, torch.tanh, operator.add, operator.mul, torch.add,
               torch.mul)


@dataclass(frozen=True)
class MatmulSpec:
    """A rank-two product ``left @ right`` with static sizes and native operand layouts."""

    m: int
    n: int
    k: int
    node: torch.fx.Node
    left: torch.fx.Node              # source of the left operand
    right: torch.fx.Node             # source of the right operand (the packed weight's get_attr when packed)
    accumulator: torch.dtype
    epilogue: bool
    transposed: tuple[bool, bool]    # (left is stored [K, M], right is stored [N, K])
    packed: bool = False             # right is a packed weight [N, K] used as deq(W)^T
    scaled: tuple | None = None      # FP8 product: (scale_a node, scale_b node, out_dtype)


def _meta(node) -> object | None:
    return node.meta.get("tensor_meta") if isinstance(node, torch.fx.Node) else None


def _transpose_source(node: torch.fx.Node) -> torch.fx.Node | None:
    """The input of a rank-two transpose node (t, .T, transpose(0, 1), permute(1, 0)), else None."""
    if node.op == "call_method" and node.target == "t":
        return node.args[0]
    if node.op == "call_function" and node.target in (torch.t,):
        return node.args[0]
    if node.op == "call_function" and node.target is getattr and node.args[1] in ("T", "mT"):
        return node.args[0]
    if node.target in ("transpose", torch.transpose) and tuple(node.args[1:3]) in ((0, 1), (1, 0), (-1, -2), (-2, -1)):
        return node.args[0]
    if node.target in ("permute", torch.permute):
        dims = node.args[1] if len(node.args) == 2 and isinstance(node.args[1], (tuple, list)) else node.args[1:]
        if tuple(dims) == (1, 0):
            return node.args[0]
    return None


def _fetch(root: torch.nn.Module | None, target: str):
    obj = root
    for part in target.split("."):
        obj = getattr(obj, part, None)
    return obj


def _packed_source(node, root: torch.nn.Module | None) -> tuple[torch.fx.Node, PackedTensor] | None:
    """(get_attr node, PackedTensor) of an ``unpack(packed, dtype)`` node, else None."""
    if isinstance(node, torch.fx.Node) and node.op == "call_function" and node.target is unpack:
        src = node.args[0]
        if isinstance(src, torch.fx.Node) and src.op == "get_attr":
            packed = _fetch(root, src.target)
            if isinstance(packed, PackedTensor):
                return src, packed
    return None


class PackedTracer(torch.fx.Tracer):
    """FX tracer that records ``PackedTensor.unpack`` as an ``unpack`` node.

    A PackedTensor reached during tracing becomes an attribute of the traced root (a get_attr
    node), so the graph refers to the packed weight instead of a decoded copy.
    """

    def create_arg(self, a):
        if isinstance(a, PackedTensor):
            names = self.__dict__.setdefault("_packed_names", {})
            if id(a) not in names:
                names[id(a)] = f"_tgm_packed_{len(names)}"
                setattr(self.root, names[id(a)], a)
            return self.create_node("get_attr", names[id(a)], (), {})
        return super().create_arg(a)

    def trace(self, root, concrete_args=None):
        tracer, original = self, PackedTensor.unpack

        def recorded_unpack(packed, dtype=None):
            return tracer.create_proxy("call_function", unpack, (packed, dtype), {})

        PackedTensor.unpack = recorded_unpack
        try:
            return super().trace(root, concrete_args)
        finally:
            PackedTensor.unpack = original


def _is_matmul(node: torch.fx.Node) -> bool:
    return ((node.op == "call_function" and (node.target in MATMUL_FUNCTIONS or
                                             (SCALED_MM is not None and node.target is SCALED_MM)))
            or (node.op == "call_method" and node.target in MATMUL_METHODS))


def _scalar_f32(node) -> bool:
    m = _meta(node)
    return m is not None and m.dtype is torch.float32 and int(torch.Size(m.shape).numel()) == 1


def _match_scaled_mm(node: torch.fx.Node) -> MatmulSpec | None:
    """``torch._scaled_mm(a, b, scale_a, scale_b[, out_dtype=...])`` with FP8 a [M, K] (row-major),
    b [K, N] (column-major, i.e. the transpose of an [N, K] row-major tensor), per-tensor fp32
    scales and a bf16 / f16 / f32 output; no bias or result scale."""
    if len(node.args) != 4 or set(node.kwargs) - {"out_dtype", "bias", "scale_result", "use_fast_accum"}:
        return None
    if node.kwargs.get("bias") is not None or node.kwargs.get("scale_result") is not None:
        return None
    left, right, sa, sb = node.args
    out, lm, rm = _meta(node), _meta(left), _meta(right)
    if out is None or lm is None or rm is None or len(lm.shape) != 2 or len(rm.shape) != 2:
        return None
    if lm.dtype not in FP8_DTYPES or rm.dtype not in FP8_DTYPES or out.dtype not in OUTPUT_DTYPES:
        return None
    if not (_scalar_f32(sa) and _scalar_f32(sb)) or lm.stride[1] != 1 or rm.stride[0] != 1:
        return None
    m, k = lm.shape
    n = rm.shape[1]
    right_src = _transpose_source(right)
    return MatmulSpec(m, n, k, node, left, right_src if right_src is not None else right, torch.float32,
                      _has_epilogue(node), (False, right_src is not None), scaled=(sa, sb, out.dtype))


def match_matmul(node: torch.fx.Node, root: torch.nn.Module | None = None) -> MatmulSpec | None:
    """Match a rank-two matrix product of a shape-propagated graph, or return None.

    ``root`` resolves the packed weights a traced graph refers to by attribute."""
    if not _is_matmul(node) or node.meta.get(KEEP):
        return None
    if SCALED_MM is not None and node.target is SCALED_MM:
        return _match_scaled_mm(node)
    if len(node.args) != 2 or node.kwargs:
        return None
    out = _meta(node)
    left, right = node.args
    lm, rm = _meta(left), _meta(right)
    if out is None or lm is None or rm is None:
        return None
    if len(lm.shape) != 2 or len(rm.shape) != 2 or len(out.shape) != 2:
        return None  # batched, broadcast or vector products keep their ordinary lowering
    if any(not isinstance(d, int) for d in (*lm.shape, *rm.shape)) or any(d <= 0 for d in (*lm.shape, *rm.shape)):
        return None
    if 0 in lm.stride or 0 in rm.stride:
        return None  # expanded (broadcast) operands
    m, k = lm.shape
    n = rm.shape[1]
    found = None
    right_src = _transpose_source(right)
    if right_src is not None:
        found = _packed_source(right_src, root)
    if found is not None:
        attr, packed = found
        if tuple(packed.shape) != (n, k) or lm.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            return None
        return MatmulSpec(m, n, k, node, left, attr, torch.float32, _has_epilogue(node), (False, True), packed=True)
    if lm.dtype not in DENSE_DTYPES or rm.dtype is not lm.dtype:
        return None  # no native ordinary kernel for this dtype
    left_src = _transpose_source(left)
    return MatmulSpec(m, n, k, node, left_src if left_src is not None else left,
                      right_src if right_src is not None else right, torch.float32, _has_epilogue(node),
                      (left_src is not None, right_src is not None))


def _has_epilogue(node: torch.fx.Node) -> bool:
    users = list(node.users)
    return len(users) == 1 and getattr(users[0], "target", None) in ELEMENTWISE


class _NativeMatmul(torch.autograd.Function):
    """``a @ b`` (a [M, K], b [K, N], bf16 or f16) on the ordinary MFMA GEMM, fp32 accumulation,
    the operands' dtype out; gradients through the same kernels."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        ctx.save_for_backward(a, b)
        return linalg.matmul(a, b, dtype=a.dtype)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        a, b = ctx.saved_tensors
        grad = grad.to(a.dtype)
        grad_a = grad_b = None
        if ctx.needs_input_grad[0]:
            grad_a = linalg.matmul_nt(grad, b, dtype=a.dtype)            # [M, N] @ [K, N]^T
        if ctx.needs_input_grad[1]:
            grad_b = linalg.matmul(a.t(), grad, dtype=b.dtype)           # [K, M] @ [M, N]
        return grad_a, grad_b


class _PackedMatmul(torch.autograd.Function):
    """``x @ deq(w)^T`` for a packed weight w [N, K] on the packed families; the gradient with
    respect to x is ``grad @ deq(w)``, run on the decoded weight."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: PackedTensor) -> torch.Tensor:
        ctx.w = w
        return linalg.matmul_nt(x, w, dtype=x.dtype if x.dtype in DENSE_DTYPES else torch.float32)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        if not ctx.needs_input_grad[0]:
            return None, None
        dt = grad.dtype if grad.dtype in DENSE_DTYPES else torch.float32
        return linalg.matmul(grad.to(dt), ctx.w.unpack(dt), dtype=grad.dtype), None


def native_matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return _NativeMatmul.apply(a, b)


def scaled_fp8_matmul(a: torch.Tensor, b_nk: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
                      out_dtype: torch.dtype) -> torch.Tensor:
    """``(a @ b_nk^T) * scale_a * scale_b`` rounded once to ``out_dtype``: FP8 a [M, K] and b_nk
    [N, K] on the FP8 GEMM.  Shapes it cannot tile (K not a multiple of 128) run the exact-width
    device GEMM, then the scale and the rounding."""
    try:
        return linalg.dense_matmul_nt(a, b_nk, out_dtype, scale_a, scale_b)
    except K.UnsupportedKernel:
        acc = linalg.matmul_nt(a, b_nk, dtype=torch.float32)
        return (acc * (scale_a * scale_b)).to(out_dtype)


def packed_matmul(x: torch.Tensor, w: PackedTensor) -> torch.Tensor:
    return _PackedMatmul.apply(x, w)


def _lower(graph: torch.fx.Graph, spec: MatmulSpec) -> None:
    node = spec.node
    with graph.inserting_before(node):
        if spec.packed:
            new = graph.call_function(packed_matmul, (node.args[0], spec.right))
        elif spec.scaled is not None:
            sa, sb, out_dtype = spec.scaled
            right = spec.right if spec.transposed[1] else graph.call_method("t", (spec.right,))
            new = graph.call_function(scaled_fp8_matmul, (spec.left, right, sa, sb, out_dtype))
        else:
            left = graph.call_method("t", (spec.left,)) if spec.transposed[0] else spec.left
            right = graph.call_method("t", (spec.right,)) if spec.transposed[1] else spec.right
            new = graph.call_function(native_matmul, (left, right))
    new.meta.update(node.meta)
    new.meta["tgm_spec"] = (spec.m, spec.n, spec.k, spec.transposed, spec.epilogue)
    node.replace_all_uses_with(new)
    graph.erase_node(node)


def lower_matmul(gm: torch.fx.GraphModule, *example_inputs) -> torch.fx.GraphModule:
    """Shape-propagate ``gm`` on ``example_inputs`` and rewrite every eligible product in place.

    Returns ``gm``; ``gm.lowered_matmuls`` lists the (m, n, k) of the rewritten products.
    """
    ShapeProp(gm).propagate(*example_inputs)
    specs = [s for s in (match_matmul(n, gm) for n in list(gm.graph.nodes)) if s is not None]
    for spec in specs:
        _lower(gm.graph, spec)
    gm.graph.eliminate_dead_code()
    gm.recompile()
    gm.lowered_matmuls = [(s.m, s.n, s.k) for s in specs]
    return gm


def trace(fn) -> torch.fx.GraphModule:
    """Trace a module or function with ``PackedTracer``."""
    tracer = PackedTracer()
    graph = tracer.trace(fn)
    return torch.fx.GraphModule(tracer.root, graph)


def trace_and_lower(fn, *example_inputs) -> torch.fx.GraphModule:
    """Trace a module or function (``trace``), then ``lower_matmul`` it."""
    return lower_matmul(trace(fn), *example_inputs)
