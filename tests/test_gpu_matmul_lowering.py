"""The ordinary MFMA GEMM and the traced-program rewrite on gfx950.

Mirrors the reference's GPU lowering tests (test/backend/test_matmul_lowering.py:70-181):
an ordinary f16 product keeps its storage dtype and matches the exact product within
rtol/atol 3e-3, gradients flow, replays with changed and misaligned inputs stay correct.
"""

import numpy as np
import pytest
import torch

import packed_oracle as O
from tinygrad_mi355x.codegen import linalg
from tinygrad_mi355x.codegen import matmul as MM
from tinygrad_mi355x.codegen.decomp.mi355x import FORMATS, PackedTensor

pytestmark = pytest.mark.gpu


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mnk", [(128, 256, 64), (200, 300, 512), (33, 1000, 192), (1, 513, 4096), (513, 7, 128)])
@pytest.mark.parametrize("out", [torch.float32, None])
def test_dense_gemm_parity(dev, dtype, mnk, out):
    """C = A @ B on the dense MFMA GEMM: B row-major (staged by the transpose kernel) and as a
    transposed view of a K-last tensor (bound directly); ragged M and N."""
    m, n, k = mnk
    rng = np.random.default_rng(m + n + k)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(dtype)
    b = torch.from_numpy(rng.standard_normal((k, n)).astype(np.float32)).to(dev).to(dtype)
    ref = f64(a) @ f64(b)
    c1 = linalg.matmul(a, b, scope="ThreadGroup", dtype=out)
    c2 = linalg.matmul(a, b.t().contiguous().t(), scope="ThreadGroup", dtype=out)
    c3 = linalg.matmul_nt(a, b.t().contiguous(), scope="ThreadGroup", dtype=out)
    assert c1.dtype is (out or torch.float32)
    for c in (c1, c2, c3):
        assert O.max_rel_err(f64(c), ref) <= 1e-2


def test_dense_gemm_one_hot_is_exact(dev):
    """One-hot rows of A pick rows of B^T exactly: operand layout, swizzle and K order line up."""
    m, n, k = 256, 512, 1024
    rng = np.random.default_rng(5)
    b = torch.from_numpy(rng.standard_normal((k, n)).astype(np.float32)).to(dev).to(torch.bfloat16)
    cols = rng.choice(k, m, replace=True)
    a = torch.zeros((m, k), dtype=torch.bfloat16, device=dev)
    a[torch.arange(m), torch.from_numpy(cols)] = 1.0
    c = linalg.matmul(a, b, scope="ThreadGroup", dtype=torch.float32)
    assert torch.equal(c, b[torch.from_numpy(cols).to(dev)].float())


def test_transpose16(dev):
    x = torch.randint(-30000, 30000, (300, 517), dtype=torch.int16, device=dev)
    view = x[:, 5:405]
    assert torch.equal(linalg.transpose16(view), view.t())


def test_ordinary_matmul_eager_gradient_and_replay(dev):
    """The rewritten f16 product keeps its dtype, matches the exact product (rtol/atol 3e-3 as
    the reference's test), gives the right gradients, and replays with changed inputs."""
    data_a = (np.arange(16 * 64, dtype=np.float32).reshape(16, 64) % 5 - 2)
    data_b = (np.arange(64 * 48, dtype=np.float32).reshape(64, 48) % 3 - 1)
    a = torch.tensor(data_a, dtype=torch.float16, device=dev)
    b = torch.tensor(data_b, dtype=torch.float16, device=dev)
    gm = MM.trace_and_lower(lambda x, y: x @ y, a, b)
    assert gm.lowered_matmuls == [(16, 48, 64)]
    out = gm(a, b)
    assert out.dtype is torch.float16
    np.testing.assert_allclose(f64(out), data_a @ data_b, rtol=3e-3, atol=3e-3)
    ga, gb = a.clone().requires_grad_(), b.clone().requires_grad_()
    linalg.fallbacks.clear()
    gm(ga, gb).float().sum().backward()
    assert not linalg.fallbacks  # the gradient products (K = 48 and 16) run zero-padded on the MFMA GEMM
    np.testing.assert_allclose(f64(ga.grad), np.ones((16, 48)) @ data_b.T, rtol=3e-3, atol=3e-3)
    np.testing.assert_allclose(f64(gb.grad), data_a.T @ np.ones((16, 48)), rtol=3e-3, atol=3e-3)
    for step in range(4):
        a2 = torch.tensor(data_a + step, dtype=torch.float16, device=dev)
        np.testing.assert_allclose(f64(gm(a2, b)), (data_a + step) @ data_b, rtol=3e-3, atol=3e-3)


@pytest.mark.parametrize("offset", [1, 3, 64])
def test_misaligned_views_are_staged(dev, offset):
    """Operands at 2-byte offsets (rows not 16-byte aligned) replay correctly through staging."""
    data_a = np.arange(16 * 64 + 128, dtype=np.float32) % 5 - 2
    data_b = (np.arange(64 * 48, dtype=np.float32).reshape(64, 48) % 3 - 1)
    b = torch.tensor(data_b, dtype=torch.float16, device=dev)
    base = torch.tensor(data_a, dtype=torch.float16, device=dev)
    gm = MM.trace_and_lower(lambda x, y: torch.relu(x @ y), base[:16 * 64].reshape(16, 64), b)
    for step in range(3):
        base = torch.tensor(data_a + step, dtype=torch.float16, device=dev)
        a = base[offset:offset + 16 * 64].reshape(16, 64)
        want = np.maximum((data_a[offset:offset + 16 * 64] + step).reshape(16, 64) @ data_b, 0)
        linalg.fallbacks.clear()
        np.testing.assert_allclose(f64(gm(a, b)), want, rtol=3e-3, atol=3e-3)
        assert not linalg.fallbacks  # staged zero-padded onto the MFMA GEMM, not the exact-width one


def test_packed_weight_product_is_not_materialised(dev):
    """``x @ w.unpack(dtype).T`` runs the packed kernels on the packed weight; the decode node is
    gone from the rewritten graph, and the result and input gradient match the oracle."""
    rng = np.random.default_rng(9)
    n, k = 384, 512
    codes = rng.integers(0, 16, (n, k)).astype(np.uint8)
    e = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.uint8)
    w = PackedTensor(torch.from_numpy(O.pack_codes(codes, FORMATS["fp4_e2m1"][0])).to(dev), "fp4_e2m1", (n, k),
                     torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu), 32)
    deq = O.dequant_f64(O.pack_codes(codes, 4), "fp4_e2m1", (n, k), O.e8m0_decode(e), 32)

    class Layer(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.w = w

        def forward(self, x):
            return x @ self.w.unpack(torch.bfloat16).t()

    x = torch.from_numpy(rng.standard_normal((40, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    gm = MM.trace_and_lower(Layer(), x)
    targets = [node.target for node in gm.graph.nodes if node.op == "call_function"]
    assert MM.packed_matmul in targets and not any(getattr(t, "__name__", "") == "unpack" for t in targets)
    xg = x.clone().requires_grad_()
    y = gm(xg)
    assert O.max_rel_err(f64(y), f64(x) @ deq.T) <= 1e-2
    y.float().sum().backward()
    assert O.max_rel_err(f64(xg.grad), np.ones((40, n)) @ deq) <= 1e-2


@pytest.mark.parametrize("k", [256, 96])
def test_scaled_fp8_product_is_lowered(dev, k):
    """A traced torch._scaled_mm runs the FP8 GEMM (K = 96 is staged zero-padded to the GEMM's
    128-element step); both match the exact fp64 product times the per-tensor scales, and
    neither falls back to the exact-width GEMM."""
    g = torch.Generator(device=dev)
    g.manual_seed(k)
    a = (torch.randn((130, k), device=dev, generator=g) * 3).to(torch.float8_e4m3fn)
    w = (torch.randn((200, k), device=dev, generator=g) * 3).to(torch.float8_e5m2)
    sa, sb = torch.tensor(0.25, device=dev), torch.tensor(1.5, device=dev)

    def f(a, w, sa, sb):
        return torch._scaled_mm(a, w.t(), sa, sb, out_dtype=torch.float32)

    # shapes are propagated on CPU copies (torch runs _scaled_mm there), the product runs on the GPU
    gm = MM.lower_matmul(MM.trace(f), *(t.cpu() for t in (a, w, sa, sb)))
    assert gm.lowered_matmuls == [(130, 200, k)]
    linalg.fallbacks.clear()
    out = gm(a, w, sa, sb)
    assert not linalg.fallbacks
    ref = a.float().cpu().numpy().astype(np.float64) @ w.float().cpu().numpy().astype(np.float64).T * 0.375
    assert out.dtype is torch.float32
    assert O.max_rel_err(out.cpu().numpy(), ref) <= 1e-2


# Products with at least one round of 256 x 256 tiles (256 CUs) and K a multiple of 128 run the
# persistent dense kernel (gemm_dense_stream): one workgroup per CU walking its tiles.
STREAM_SHAPES = [(4096, 4096, 256), (4000, 4200, 384), (8192, 4352, 128)]


@pytest.mark.parametrize("mnk", STREAM_SHAPES)
def test_dense_stream_one_hot_is_exact(dev, mnk):
    """One-hot rows of A pick rows of B exactly in every output tile of the persistent kernel
    (ragged edges, several tiles per workgroup, bf16 and f32 outputs): operand layout, swizzle,
    K order, tile walk and epilogue line up."""
    from tinygrad_mi355x.renderer.matrix import GEMM_DENSE_STREAM, dense_kernel

    m, n, k = mnk
    assert dense_kernel(m, n, k) is GEMM_DENSE_STREAM
    rng = np.random.default_rng(m + k)
    b = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    cols = torch.from_numpy(rng.integers(0, k, m)).to(dev)
    a = torch.zeros((m, k), dtype=torch.bfloat16, device=dev)
    a[torch.arange(m, device=dev), cols] = 1.0
    want = b.t()[cols]  # [m, n]: row i of C is column cols[i] of B^T
    for out in (torch.float32, torch.bfloat16):
        c = linalg.dense_matmul_nt(a, b, out)
        assert torch.equal(c, want.to(out)), out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mnk", STREAM_SHAPES[:2])
def test_dense_stream_parity(dev, dtype, mnk):
    """Random operands against the fp64 product (bf16 / f16 products are exact in fp32; only the
    summation order differs), A as a strided view (row stride > K), three output dtypes."""
    m, n, k = mnk
    rng = np.random.default_rng(n + k)
    a_full = torch.from_numpy(rng.standard_normal((m, k + 64)).astype(np.float32)).to(dev).to(dtype)
    a = a_full[:, 32:32 + k]
    b = torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).to(dev).to(dtype)
    rows = torch.from_numpy(rng.choice(m, 256, replace=False)).to(dev)
    a_rows, b64 = f64(a[rows]), f64(b)
    ref = a_rows @ b64.T
    bound = k * 2.0 ** -23 * (np.abs(a_rows) @ np.abs(b64).T)  # fp32 sums of exact products
    for out in (torch.float32, torch.bfloat16, torch.float16):
        c = linalg.dense_matmul_nt(a, b, out)
        got = f64(c[rows])
        assert O.max_rel_err(got, ref) <= 1e-2, out
        if out is torch.float32:
            assert bool((np.abs(got - ref) <= bound).all())
