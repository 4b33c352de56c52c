"""Conservative recognition of rank-two matrix products in traced programs (CPU).

Mirrors the reference's scheduled-matmul tests (test/backend/test_matmul_lowering.py:24-54):
an exact row-major product is recognised with its sizes and operand slots; transposes,
epilogues and dtypes are preserved; broadcast products, extra outputs and pinned nodes keep
their ordinary lowering.  Shapes are propagated on meta tensors, so nothing is computed.
"""

import pytest
import torch

from tinygrad_mi355x.codegen import matmul as MM


def meta(*shape, dtype=torch.float16):
    return torch.empty(shape, dtype=dtype, device="meta")


def specs(fn, *inputs):
    gm = MM.trace(fn)
    from torch.fx.passes.shape_prop import ShapeProp

    ShapeProp(gm).propagate(*inputs)
    found = [MM.match_matmul(n, gm) for n in gm.graph.nodes if MM._is_matmul(n)]
    return gm, found


def test_recognizes_exact_row_major_matrix():
    gm, found = specs(lambda a, b: a @ b, meta(16, 32), meta(32, 48))
    (spec,) = found
    assert (spec.m, spec.n, spec.k) == (16, 48, 32)
    assert (spec.left.name, spec.right.name) == ("a", "b")
    assert spec.transposed == (False, False) and not spec.epilogue and not spec.packed


@pytest.mark.parametrize("kind", ["transposed", "activated", "bfloat16", "right_transposed"])
def test_recognizes_native_matrix_semantics(kind):
    dtype = torch.bfloat16 if kind == "bfloat16" else torch.float16
    if kind == "transposed":
        fn, inputs = (lambda a, b: a.t() @ b), (meta(32, 16), meta(32, 48))
    elif kind == "right_transposed":
        fn, inputs = (lambda a, b: torch.matmul(a, b.transpose(0, 1))), (meta(16, 32), meta(48, 32))
    elif kind == "activated":
        fn, inputs = (lambda a, b: torch.relu(a @ b)), (meta(16, 32), meta(32, 48))
    else:
        fn, inputs = (lambda a, b: a.mm(b)), (meta(16, 32, dtype=dtype), meta(32, 48, dtype=dtype))
    _, (spec,) = specs(fn, *inputs)
    assert (spec.m, spec.n, spec.k) == (16, 48, 32)
    assert spec.transposed == (kind == "transposed", kind == "right_transposed")
    assert spec.epilogue == (kind == "activated")
    assert spec.left.meta["tensor_meta"].dtype is dtype


def test_rejects_broadcast_batched_and_second_output():
    # a batched (rank-three) product and an expanded operand keep their ordinary lowering
    _, found = specs(lambda a, b: a @ b, meta(4, 16, 32), meta(32, 48))
    assert found == [None]
    _, found = specs(lambda a, b: a.expand(16, 32) @ b, meta(1, 32), meta(32, 48))
    assert found == [None]
    # a product that also writes a second tensor (out=) is not replaced
    _, found = specs(lambda a, b, c: torch.matmul(a, b, out=c), meta(16, 32), meta(32, 48), meta(16, 48))
    assert found == [None]


def test_rejects_pinned_nodes_and_dtypes_without_a_native_kernel():
    gm = MM.trace(lambda a, b: a @ b)
    for node in gm.graph.nodes:
        if MM._is_matmul(node):
            node.meta[MM.KEEP] = True
    from torch.fx.passes.shape_prop import ShapeProp

    ShapeProp(gm).propagate(meta(16, 32), meta(32, 48))
    assert [MM.match_matmul(n, gm) for n in gm.graph.nodes if MM._is_matmul(n)] == [None]
    for dtype in (torch.float32, torch.float64, torch.int8):
        _, found = specs(lambda a, b: a @ b, meta(16, 32, dtype=dtype), meta(32, 48, dtype=dtype))
        assert found == [None]
    _, found = specs(lambda a, b: a @ b, meta(16, 32), meta(32, 48, dtype=torch.bfloat16))
    assert found == [None]  # mixed operand dtypes


def test_lowering_replaces_products_and_keeps_the_rest():
    def fn(a, b, c):
        return torch.relu(a @ b) + (c @ c.t()).sum() + torch.bmm(a[None], b[None])[0]

    gm = MM.lower_matmul(MM.trace(fn), meta(16, 32), meta(32, 48), meta(24, 64))
    targets = [n.target for n in gm.graph.nodes if n.op == "call_function"]
    assert targets.count(MM.native_matmul) == 2
    assert torch.bmm in targets  # batched product untouched
    assert sorted(gm.lowered_matmuls) == [(16, 48, 32), (24, 24, 64)]


def test_recognizes_fp8_scaled_products():
    """torch._scaled_mm with per-tensor fp32 scales and a bf16 / f16 / f32 output is an FP8
    product on the FP8 GEMM; an fp8 output or a bias keeps torch's lowering (CPU tensors: torch
    runs _scaled_mm here for shape propagation)."""
    a = torch.randn(16, 128).to(torch.float8_e4m3fn)
    w = torch.randn(48, 128).to(torch.float8_e5m2)
    sa, sb = torch.tensor(0.5), torch.tensor(2.0)

    def f(a, w, sa, sb):
        return torch._scaled_mm(a, w.t(), sa, sb, out_dtype=torch.bfloat16)

    gm, (spec,) = specs(f, a, w, sa, sb)
    assert (spec.m, spec.n, spec.k) == (16, 48, 128)
    assert spec.right.name == "w" and spec.transposed == (False, True)
    assert spec.scaled[2] is torch.bfloat16 and spec.scaled[0].name == "sa"
    lowered = MM.lower_matmul(MM.trace(f), a, w, sa, sb)
    assert lowered.lowered_matmuls == [(16, 48, 128)]
    assert any(n.target is MM.scaled_fp8_matmul for n in lowered.graph.nodes)
    _, found = specs(lambda a, w, sa, sb: torch._scaled_mm(a, w.t(), sa, sb), a, w.to(torch.float8_e4m3fn), sa, sb)
    assert found == [None]  # FP8 output
    bias = torch.zeros(48, dtype=torch.bfloat16)
    _, found = specs(lambda a, w, sa, sb: torch._scaled_mm(a, w.t(), sa, sb, bias=bias, out_dtype=torch.bfloat16),
                     a, w.to(torch.float8_e4m3fn), sa, sb)
    assert found == [None]
