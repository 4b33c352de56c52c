"""The packed path on the plugin's own buffers, end to end on gfx950 (no torch tensors).

The reference's standalone chain is ``PackedTensor.matmul`` -> LinAlg table -> launch
(codegen/decomp/dx12.py:108-112, codegen/linalg.py:136-298).  Here ``codegen/program.py``
runs it over ``MI355XBuffer`` storage from the device allocator, on the device's stream:
decode bit-exact against the oracle, products within the stated tolerance of the oracle's
exact fp64 product.
"""

import numpy as np
import pytest

import packed_oracle as O
from tinygrad_mi355x.codegen import program as P
from tinygrad_mi355x.runtime import ops_mi355x as R

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture(scope="module")
def device():
    d = R.get_device("MI355X")
    yield d
    d.synchronize()


def upload(dev, arr: np.ndarray):
    buf = dev.allocator.alloc(max(arr.nbytes, 1))
    dev.allocator._copyin(buf, memoryview(np.ascontiguousarray(arr)).cast("B"))
    return buf


def download(dev, m: P.Matrix, np_dtype) -> np.ndarray:
    out = np.empty(int(np.prod(m.shape)), np_dtype)
    m.buf.dev.synchronize()
    dev.allocator._copyout(memoryview(out).cast("B"), m.buf)
    return out.reshape(m.shape)


def packed(dev, fmt, n, k, rng, scaled=True):
    bits = O.bits_of(fmt)
    codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint8)
    data = O.pack_codes(codes, bits)
    scales = None
    e = None
    if scaled:
        e = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.uint8)
        scales = P.Matrix(upload(dev, e), "float8_e8m0fnu", e.shape)
    w = P.PackedBuffer(upload(dev, data), fmt, (n, k), scales, 32)
    deq = O.dequant_f64(data, fmt, (n, k), None if e is None else O.e8m0_decode(e), 32)
    return w, data, e, deq


def bf16_matrix(dev, rng, m, k):
    xb = O.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    return P.Matrix(upload(dev, xb), "bfloat16", (m, k)), O.bf16_to_f32(xb).astype(np.float64)


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e3m2", "int4"])
def test_unpack_on_plugin_buffers_is_bit_exact(device, fmt):
    rng = np.random.default_rng(1)
    w, data, e, _ = packed(device, fmt, 64, 256, rng, scaled=fmt != "int4")
    got = download(device, w.unpack(), np.int32 if fmt == "int4" else np.float32)
    want = O.unpack(data, fmt, (64, 256), None if e is None else O.e8m0_decode(e), 32)
    assert np.array_equal(got.view(np.uint32), np.asarray(want).view(np.uint32))


@pytest.mark.parametrize("m", [1, 4, 48])
def test_weight_products_on_plugin_buffers(device, m):
    """FP4 + E8M0/32 weight x bf16 activations: GEMV (M <= 16) and the dequant GEMM."""
    rng = np.random.default_rng(m)
    w, _, _, deq = packed(device, "fp4_e2m1", 1024, 4096, rng)
    x, xf = bf16_matrix(device, rng, m, 4096)
    y = P.matmul_nt(x, w)  # [M, N] fp32
    assert y.shape == (m, 1024) and y.dtype == "float32"
    assert O.max_rel_err(download(device, y, np.float32), xf @ deq.T) <= TOL


def test_matvec_and_timed_program(device):
    """matvec is a one-row product; a program called with wait returns its seconds."""
    rng = np.random.default_rng(9)
    w, _, _, deq = packed(device, "fp4_e2m1", 14336, 4096, rng)
    x, xf = bf16_matrix(device, rng, 1, 4096)
    v = P.Matrix(x.buf, "bfloat16", (4096,))
    y = P.matvec(w, v, "bfloat16")
    assert y.shape == (14336,)
    got = O.bf16_to_f32(download(device, y, np.uint16)).astype(np.float64)
    assert O.max_rel_err(got, deq @ xf[0]) <= TOL
    prog = P.weight_program(w.desc(), 1, "bfloat16", 4096, "bfloat16", 14336)
    out = device.allocator.alloc(14336 * 2)
    seconds = prog(out, w.data, x.buf, wait=True)
    assert isinstance(seconds, float) and 0 < seconds < 1


@pytest.mark.parametrize("fa,fb", [("fp4_e2m1", "fp4_e2m1"), ("fp6_e2m3", "fp4_e2m1"), ("fp6_e3m2", "fp6_e3m2")])
def test_packed_pairs_on_plugin_buffers(device, fa, fb):
    rng = np.random.default_rng(len(fa) + len(fb))
    a, _, _, deq_a = packed(device, fa, 256, 512, rng)
    b, _, _, deq_b = packed(device, fb, 192, 512, rng, scaled=fb != "fp6_e3m2")
    c = P.matmul_nt(a, b)
    assert O.max_rel_err(download(device, c, np.float32), deq_a @ deq_b.T) <= TOL


def test_dense_pair_on_plugin_buffers(device):
    rng = np.random.default_rng(4)
    a, af = bf16_matrix(device, rng, 130, 256)
    b, bf = bf16_matrix(device, rng, 260, 256)
    c = P.matmul_nt(a, b, "float32")
    assert O.max_rel_err(download(device, c, np.float32), af @ bf.T) <= TOL
