"""GPU parity of the matrix path (gfx950 kernels through the C ABI) vs the oracle.

Known-answer cases mirror the reference's test_linalg.py / test_packed.py; the random
cases compare against the oracle's exactly dequantised weights with an fp64 product,
max elementwise relative error <= 1e-2 (see packed_oracle.max_rel_err).
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import packed_oracle as O
from tinygrad_mi355x.codegen import linalg
from tinygrad_mi355x.codegen.decomp.mi355x import FORMATS, PackedTensor, matmul as decomp_matmul, quantize_mx
from tinygrad_mi355x.codegen.linalg import matmul, matmul_nt, matvec

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
TOL = 1e-2
TORCH_DT = {"int8": torch.int8, "uint8": torch.uint8, "int32": torch.int32, "int64": torch.int64,
            "uint64": torch.uint64, "float64": torch.float64, "float16": torch.float16, "float32": torch.float32}


def bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def host_dequant_rows(p: PackedTensor, rows) -> np.ndarray:
    """Exact fp64 values of the selected rows of a 2-D MX PackedTensor, decoded by the oracle from
    the host copy of its packed bytes and E8M0 scale bytes (no device decode involved)."""
    n, k = p.shape
    data = p.data.cpu().numpy().reshape(n, -1)[rows].reshape(-1)
    e = p.scales.view(torch.uint8).cpu().numpy()[rows]
    return O.dequant_f64(data, p.format, (len(rows), k), O.e8m0_decode(e), p.block_size)


def stratified(rng, size: int, per_band: int, band: int = 32) -> np.ndarray:
    """Sorted indices with ``per_band`` distinct random picks in every ``band``-wide band of
    [0, size) (fewer in a short last band): sampled rows x sampled columns then hold outputs of
    every 32 x 32 MFMA output tile, so no workgroup, wave or tile-order slot goes unchecked."""
    picks = [start + rng.choice(min(band, size - start), min(per_band, size - start), replace=False)
             for start in range(0, size, band)]
    return np.sort(np.concatenate(picks))


def test_stratified_covers_every_band():
    rng = np.random.default_rng(0)
    idx = stratified(rng, 14336, 2)
    assert len(idx) == 2 * 448 and len(np.unique(idx)) == len(idx)
    assert np.array_equal(np.bincount(idx // 32, minlength=448), np.full(448, 2))
    assert set(np.unique(stratified(rng, 100, 1) // 32)) == {0, 1, 2, 3}


# ----------------------------------------------------------------------------- known answers
def test_scales_stay_with_k_blocks(dev):
    case = GOLDEN["scales_stay_with_k_blocks"]
    packed = PackedTensor(torch.tensor(case["data"], dtype=torch.uint8, device=dev), case["format"], tuple(case["shape"]),
                          torch.tensor(case["scales"], device=dev), block_size=case["block_size"])
    rhs = torch.tensor(case["rhs"], device=dev)
    assert decomp_matmul(packed, rhs).tolist() == case["expected"]
    assert matmul(packed, rhs.float()).tolist() == case["expected"]


def test_double_block_scales_matmul(dev):
    case = GOLDEN["double_block_scales"]
    packed = PackedTensor(torch.tensor(case["data"], dtype=torch.uint8, device=dev), case["format"], tuple(case["shape"]),
                          torch.tensor(case["scales"], dtype=torch.float64, device=dev), block_size=case["block_size"])
    out = decomp_matmul(packed, torch.tensor(case["rhs"], device=dev))
    assert out.dtype is torch.float64 and out.tolist() == case["expected"]
    assert matmul(packed, torch.tensor(case["rhs"], device=dev)).tolist() == case["expected"]


def test_readme_uint4_matmul_and_matvec(dev):
    case = GOLDEN["readme_uint4"]
    packed = PackedTensor(torch.tensor(case["data"], dtype=torch.uint8, device=dev), "uint4", tuple(case["shape"]))
    assert matmul(packed, torch.tensor(case["column"], device=dev)).tolist() == case["matmul"]
    assert matvec(packed, torch.tensor(case["vector"], device=dev)).tolist() == case["matvec"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2, torch.int8, torch.uint8])
def test_matrix_tails(dev, dtype):
    """Non-tile dimensions with exact integer arithmetic (test_linalg.py:11-20)."""
    a = [[(i + k) % 5 for k in range(19)] for i in range(17)]
    b = [[(k + j) % 3 for j in range(21)] for k in range(19)]
    expected = [[sum(a[i][k] * b[k][j] for k in range(19)) for j in range(21)] for i in range(17)]
    ta = torch.tensor(a, dtype=torch.float32).to(dtype).to(dev)
    tb = torch.tensor(b, dtype=torch.float32).to(dtype).to(dev)
    assert matmul(ta, tb).tolist() == expected


def test_fp16_inputs_keep_fp32_accumulation(dev):
    case = GOLDEN["fp16_accumulation"]
    m = torch.tensor(case["matrix"], dtype=torch.float16, device=dev)
    v = torch.tensor(case["vector"], dtype=torch.float16, device=dev)
    result = matvec(m, v)
    assert result.dtype is torch.float32 and result.tolist() == case["expected"]


@pytest.mark.parametrize("case", GOLDEN["wide_matrix_fallback"]["cases"])
def test_wide_matrix_fallback(dev, case):
    dt = TORCH_DT[case["dtype"]]
    a = torch.tensor([case["values"]], dtype=dt, device=dev)
    b = torch.tensor([[1], [1], [1]], dtype=dt, device=dev)
    result = matmul(a, b)
    assert result.dtype is dt and result.tolist() == [[case["expected"]]]


@pytest.mark.parametrize("case", GOLDEN["packed_integer_precision"]["cases"])
def test_packed_integer_matmul_precision(dev, case):
    dt = TORCH_DT[case["dtype"]]
    weights = PackedTensor(torch.tensor([case["byte"]], dtype=torch.uint8, device=dev), case["format"], (1, 2))
    output = weights.matmul(torch.tensor([[x] for x in case["values"]], dtype=dt, device=dev))
    assert output.dtype is dt and output.tolist() == [[case["expected"]]]


@pytest.mark.parametrize("scope", ["auto", "tiled"])
@pytest.mark.parametrize("case", GOLDEN["accumulator_width"]["cases"])
def test_matrix_product_uses_accumulator_width(dev, scope, case):
    dt = TORCH_DT[case["dtype"]]
    values = case["values"]
    result = matmul(torch.tensor([values], dtype=dt, device=dev), torch.tensor([[x] for x in values], dtype=dt, device=dev),
                    scope=scope)
    assert result.dtype is {"int32": torch.int32, "uint32": torch.uint32}[case["acc"]]
    assert result.tolist() == [[sum(x * x for x in values)]]


def test_explicit_scope_without_native_kernel_raises(dev):
    a = torch.ones((4, 4), dtype=torch.float64, device=dev)
    with pytest.raises(RuntimeError, match="candidate rejected"):
        matmul(a, a, scope="Wave")


# ----------------------------------------------------------------------------- GEMV family
def make_weight(dev, fmt, n, k, scale_kind, rng, bs=32):
    bits = FORMATS[fmt][0]
    codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint8)
    data = torch.from_numpy(O.pack_codes(codes, bits)).to(dev)
    nb = (k + bs - 1) // bs
    if scale_kind == "e8m0":
        e = (127 + rng.integers(-4, 3, (n, nb))).astype(np.uint8)
        scales = torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu)
        s_np = O.e8m0_decode(e)
    elif scale_kind == "f16":
        s_np = rng.uniform(0.005, 0.02, (n, nb)).astype(np.float16)
        scales = torch.from_numpy(s_np).to(dev)
    else:
        scales, s_np = None, None
    w = PackedTensor(data, fmt, (n, k), scales, bs)
    deq = O.dequant_f64(O.pack_codes(codes, bits), fmt, (n, k), s_np, bs)
    return w, deq


@pytest.mark.parametrize("fmt,scale_kind", [("fp4_e2m1", "e8m0"), ("fp6_e2m3", "e8m0"), ("fp4_e2m1", None)])
@pytest.mark.parametrize("nkm,slices", [((1000, 4096, 8), 2), ((4096, 14336, 8), 7), ((300, 14336, 16), 7),
                                        ((4100, 2048, 5), 4), ((64, 1024, 1), 8), ((28672, 2048, 8), 2)])
def test_dec_gemv_parts(dev, fmt, scale_kind, nkm, slices):
    """K-slice partial GEMV (tgm_dec_gemv_parts): part z is x[:, K_z] . deq(W[:, K_z])^T over the
    z-th of ``slices`` equal K slices, each within the GEMV tolerance of the oracle's product over
    that slice, and their sum within it of the whole product (exact-shape and guarded kernels,
    ragged N, 1-16 activation rows)."""
    from tinygrad_mi355x.runtime import kernels as K
    n, k, m = nkm
    rng = np.random.default_rng(n + k + m + slices)
    w, deq = make_weight(dev, fmt, n, k, scale_kind, rng)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    parts = torch.full((slices, m, n), float("nan"), dtype=torch.float32, device=dev)
    K.call("tgm_dec_gemv_parts", w.data.data_ptr(), K.FORMAT_IDS[fmt], n, k, K.ptr(w.scales),
           K.dtype_id(w.scales.dtype) if w.scales is not None else -1, w.block_size, x.data_ptr(),
           K.dtype_id(torch.bfloat16), m, k, parts.data_ptr(), n, slices, torch.cuda.current_stream().cuda_stream)
    xs = x.float().cpu().numpy().astype(np.float64)
    got = parts.cpu().numpy().astype(np.float64)
    ks = k // slices
    for z in range(slices):
        ref = xs[:, z * ks:(z + 1) * ks] @ deq[:, z * ks:(z + 1) * ks].T
        assert O.max_rel_err(got[z], ref) <= TOL, z
    assert O.max_rel_err(got.sum(0), xs @ deq.T) <= TOL


def test_dec_gemv_parts_rejects_bad_slices(dev):
    """K must split into slices of whole 128-element super-steps; INT4 weights are not taken."""
    from tinygrad_mi355x.runtime import kernels as K
    rng = np.random.default_rng(5)
    w, _ = make_weight(dev, "fp4_e2m1", 64, 1024, "e8m0", rng)
    x = torch.zeros((2, 1024), dtype=torch.bfloat16, device=dev)
    parts = torch.empty((3, 2, 64), dtype=torch.float32, device=dev)
    args = (w.data.data_ptr(), K.FORMAT_IDS["fp4_e2m1"], 64, 1024, w.scales.data_ptr(), K.dtype_id(w.scales.dtype), 32,
            x.data_ptr(), K.dtype_id(torch.bfloat16), 2, 1024, parts.data_ptr(), 64)
    with pytest.raises(ValueError):
        K.call("tgm_dec_gemv_parts", *args, 3, torch.cuda.current_stream().cuda_stream)
    wi, _ = int4_weight(dev, "int4", 64, 1024, torch.float16, 32, rng)
    xi = torch.zeros((2, 1024), dtype=torch.float16, device=dev)
    with pytest.raises(K.UnsupportedKernel):
        K.call("tgm_dec_gemv_parts", wi.data.data_ptr(), K.FORMAT_IDS["int4"], 64, 1024, wi.scales.data_ptr(),
               K.dtype_id(torch.float16), 32, xi.data_ptr(), K.dtype_id(torch.float16), 2, 1024, parts.data_ptr(), 64,
               2, torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("nk", [(256, 512), (200, 384), (14336 // 8, 4096)])
def test_gemv_mx_parity(dev, fmt, m, nk):
    """Family 1 fast path: FP4/FP6 + E8M0/32, bf16 activations, bf16 out."""
    n, k = nk
    rng = np.random.default_rng(n * 31 + k + m)
    w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    y = matmul(w, x.t(), dtype=torch.bfloat16)  # [N, M] = W @ X^T
    assert y.shape == (n, m) and y.dtype is torch.bfloat16
    ref = O.matmul_reference(deq, bf16_np(x).T)
    assert O.max_rel_err(bf16_np(y), ref) <= TOL
    y2 = matmul_nt(x, w, dtype=torch.float32)  # [M, N]
    assert O.max_rel_err(y2.cpu().numpy(), ref.T) <= TOL


@pytest.fixture(scope="module")
def fp4_decode_weight_14336x4096(dev):
    """The FP4 decode weight at its full size, drawn in the documented order with seed 0:
    codes = integers(0, 16, (14336, 4096)) (all 16 E2M1 codes, -0 included), E8M0 bytes
    127 + integers(-4, 3, (14336, 128)).  Returns the device PackedTensor, the fp64 values
    dequantised on the host from the host's own codes, and the generator, positioned where the
    activation draw follows."""
    n, k = 14336, 4096
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (n, k)).astype(np.uint8)
    e = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.uint8)
    data = O.pack_codes(codes, 4)
    w = PackedTensor(torch.from_numpy(data).to(dev), "fp4_e2m1", (n, k),
                     torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu), 32)
    return w, O.dequant_f64(data, "fp4_e2m1", (n, k), O.e8m0_decode(e), 32), rng.bit_generator.state


@pytest.mark.parametrize("m", [1, 4, 16])
def test_gemv_fp4_decode_full_shape_against_oracle(dev, fp4_decode_weight_14336x4096, m):
    """The benchmarked decode GEMV at its own shape: W FP4 E2M1 + E8M0/32 [14336, 4096], X bf16
    [M, 4096] ~ N(0, 1) (drawn after W), bf16 out.  Every one of the M x 14336 outputs is held to
    max relative error 1e-2 against the fp64 product of the host-dequantised weight (M = 1 runs
    the row-streaming kernel with its full 1792-wave grid, M = 4 the row-quad kernel, M = 16 the
    streaming MFMA GEMV)."""
    w, deq, state = fp4_decode_weight_14336x4096
    rng = np.random.default_rng(0)
    rng.bit_generator.state = state
    x_np = rng.standard_normal((m, 4096)).astype(np.float32)
    x = torch.from_numpy(x_np).to(dev).to(torch.bfloat16)
    y = matmul_nt(x, w, dtype=torch.bfloat16)
    assert y.shape == (m, 14336) and y.dtype is torch.bfloat16
    ref = bf16_np(x).astype(np.float64) @ deq.T
    assert O.max_rel_err(bf16_np(y), ref) <= TOL
    # the same launch again on the same inputs is bit-identical (no run-to-run order change)
    assert torch.equal(matmul_nt(x, w, dtype=torch.bfloat16), y)


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e3m2"])
@pytest.mark.parametrize("nkm", [(12288, 2048, 1), (6144, 4096, 4), (4096, 14336, 1), (2048, 3584, 2),
                                 (256, 14336, 16), (1000, 4096, 16), (64, 1536, 7), (4096, 14336, 8),
                                 (512, 12160, 12), (12288, 4096, 5), (13000, 2048, 9), (14336, 4096, 12),
                                 (28700, 1024, 16), (28672, 2048, 8)])
def test_gemv_mx_launch_shapes(dev, fmt, nkm):
    """Every workgroup shape of the streaming GEMV (8x1 from 1792 tiles on, 4x2, 2x4, 1x8 tiles x
    K slices), exact and guarded slices, ragged N, activations staged in LDS and in the load ring
    (M x K too large for LDS: the decoder's down projection at 8 rows, and per-dword scales with
    guarded slices)."""
    n, k, m = nkm
    rng = np.random.default_rng(n + k + m)
    w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    y = matmul_nt(x, w, dtype=torch.bfloat16)
    ref = bf16_np(x).astype(np.float64) @ deq.T
    assert O.max_rel_err(bf16_np(y), ref) <= TOL


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3"])
def test_gemv_e8m0_extreme_scales(dev, fmt):
    """E8M0 bytes at the ends of the range: 255 is NaN and poisons its rows; 1..3 give
    bf16 values down to 2^-128, which the MFMA path must keep (no flush to zero)."""
    n, k = 48, 1024
    rng = np.random.default_rng(11)
    bits = FORMATS[fmt][0]
    codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint8)
    e = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.uint8)
    e[3, 5] = 255
    e[10, :] = 1  # whole row at the bottom of the range
    e[11, ::2] = 2
    e[12, 7] = 3
    data = O.pack_codes(codes, bits)
    w = PackedTensor(torch.from_numpy(data).to(dev), fmt, (n, k), torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu), 32)
    x = torch.from_numpy(rng.standard_normal((2, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    y = matmul_nt(x, w, dtype=torch.float32).cpu().numpy()  # [2, n]
    deq = O.dequant_f64(data, fmt, (n, k), O.e8m0_decode(e), 32)
    ref = bf16_np(x).astype(np.float64) @ deq.T
    assert np.array_equal(np.isnan(y), np.isnan(ref)) and np.isnan(y[:, 3]).all()
    ok = ~np.isnan(ref)
    for row in (10, 11, 12):  # tiny rows: relative error of the row itself
        r = ref[:, row]
        assert np.abs(y[:, row] - r).max() <= 1e-2 * np.abs(r).max()
    assert O.max_rel_err(np.where(ok, y, 0), np.where(ok, ref, 0)) <= TOL


@pytest.mark.parametrize("scale_kind", ["e8m0", "none"])
@pytest.mark.parametrize("nkm", [(37, 2048, 2), (250, 4096, 3), (1000, 6144, 4), (4100, 8192, 4), (1792, 4096, 2),
                                 (8192, 2048, 3), (14336, 8192, 2)])
def test_gemv_row_quads(dev, scale_kind, nkm):
    """2 <= M <= 4 FP4 GEMVs with K a multiple of 2048 up to 8192 run the row-quad kernel (four
    weight rows and the activation rows share K positions in one bf16 MFMA): ragged N (rows past
    N are clamped and not stored), every K instantiation, workgroups of 8, 16, 28 and 56 rows
    (chosen from N and the CU count), scaled and unscaled weights; a second launch on the same
    inputs is bit-identical."""
    n, k, m = nkm
    rng = np.random.default_rng(n + 7 * k + m)
    w, deq = make_weight(dev, "fp4_e2m1", n, k, scale_kind, rng)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    y = matmul_nt(x, w, dtype=torch.bfloat16)
    ref = bf16_np(x).astype(np.float64) @ deq.T
    assert O.max_rel_err(bf16_np(y), ref) <= TOL
    assert torch.equal(matmul_nt(x, w, dtype=torch.bfloat16), y)


def test_gemv_row_quads_one_hot_and_strides(dev):
    """One-hot activation rows recover columns of deq(W) exactly at the chunk, instruction and
    K-slice edges of K = 4096; through the C ABI, activations with ldx > K and outputs with
    ldy > N in f32 and f16 (the columns past N keep their contents)."""
    from tinygrad_mi355x.runtime import kernels as K

    n, k = 70, 4096
    rng = np.random.default_rng(3)
    w, deq = make_weight(dev, "fp4_e2m1", n, k, "e8m0", rng)
    cols = [0, 31, 32, 511, 512, 1023, 1024, 2047, 2048, 3071, 3072, 4095]
    for start in range(0, len(cols), 4):
        sel = cols[start:start + 4]
        x = torch.zeros((len(sel), k), dtype=torch.bfloat16, device=dev)
        for i, j in enumerate(sel):
            x[i, j] = 1.0
        y = matmul_nt(x, w, dtype=torch.float32).cpu().numpy()
        assert np.array_equal(y, deq[:, sel].T.astype(np.float32))
    m, ldx, ldy = 3, k + 64, n + 5
    xs = torch.from_numpy(rng.standard_normal((m, ldx)).astype(np.float32)).to(dev).to(torch.bfloat16)
    ref = bf16_np(xs[:, :k]).astype(np.float64) @ deq.T
    for tdt in (torch.float32, torch.float16):
        y = torch.full((m, ldy), 7.0, dtype=tdt, device=dev)
        K.call("tgm_gemv", w.data.data_ptr(), K.FORMAT_IDS["fp4_e2m1"], n, k, K.ptr(w.scales),
               K.dtype_id(w.scales.dtype), 32, xs.data_ptr(), K.dtype_id(xs.dtype), m, ldx, y.data_ptr(),
               K.dtype_id(tdt), ldy, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert O.max_rel_err(y[:, :n].float().cpu().numpy(), ref) <= TOL
        assert bool((y[:, n:] == 7.0).all())


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
def test_gemv_one_hot_recovers_dequantised_weights_exactly(dev, fmt):
    """x = e_j selects column j of deq(W): the fast path's in-register dequant must be exact."""
    n, k = 64, 256
    rng = np.random.default_rng(5)
    w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
    cols = [0, 1, 7, 31, 32, 100, 255]
    x = torch.zeros((len(cols), k), dtype=torch.bfloat16, device=dev)
    for i, j in enumerate(cols):
        x[i, j] = 1.0
    y = matmul_nt(x, w, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(y, deq[:, cols].T.astype(np.float32))


@pytest.mark.parametrize("fmt", list(FORMATS))
@pytest.mark.parametrize("scale_kind", ["none", "f16", "e8m0"])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16, torch.float32])
def test_gemv_general_parity(dev, fmt, scale_kind, xdt):
    n, k, m = 96, 200, 3
    rng = np.random.default_rng(17)
    w, deq = make_weight(dev, fmt, n, k, scale_kind, rng)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(xdt)
    y = matmul_nt(x, w, dtype=torch.float32)
    ref = O.matmul_reference(x.float().cpu().numpy(), deq.T)
    assert O.max_rel_err(y.cpu().numpy(), ref) <= TOL


def test_int4_gemv_4096x4096_shape(dev):
    """INT4 g32 fp16-scale GEMV, N=K=4096, x fp16 [1,4096] -> fp16."""
    rng = np.random.default_rng(0)
    x_np = rng.standard_normal((1, 4096)).astype(np.float16)
    codes = rng.integers(-8, 8, (4096, 4096))
    scales_np = rng.uniform(0.005, 0.02, (4096, 128)).astype(np.float16)
    data = O.pack_codes((codes & 0xF).astype(np.uint8), 4)
    w = PackedTensor(torch.from_numpy(data).to(dev), "int4", (4096, 4096), torch.from_numpy(scales_np).to(dev), 32)
    x = torch.from_numpy(x_np).to(dev)
    y = matvec(w, x[0], output_dtype=torch.float16)
    deq = O.dequant_f64(data, "int4", (4096, 4096), scales_np, 32)
    ref = deq @ x_np[0].astype(np.float64)
    assert y.dtype is torch.float16 and O.max_rel_err(y.float().cpu().numpy(), ref) <= TOL


def int4_weight(dev, fmt, n, k, sdt, bs, rng):
    """Random INT4/UINT4 weight with scales of dtype ``sdt`` (None: unscaled) per ``bs``."""
    codes = rng.integers(0, 16, (n, k)).astype(np.uint8)
    data = O.pack_codes(codes, 4)
    scales = s_np = None
    if sdt is not None:
        s_np = rng.uniform(0.005, 0.02, (n, k // bs)).astype(np.float32)
        scales = torch.from_numpy(s_np).to(dev).to(sdt)
        s_np = scales.float().cpu().numpy()  # the values the device holds
    w = PackedTensor(torch.from_numpy(data).to(dev), fmt, (n, k), scales, bs)
    return w, O.dequant_f64(data, fmt, (n, k), s_np, bs)


@pytest.mark.parametrize("nkm", [(640, 4096, 4), (640, 4096, 8), (384, 4096, 16), (256, 6144, 12)])
def test_gemv_int4_mfma_staging_passes(dev, nkm):
    """The f16-MFMA INT4 GEMV stages X in LDS in 2, 8 or 16 straight-line passes and a loop
    beyond: 4 and 8 rows (8-pass variant), 16 rows (16 passes), 12 x 6144 (16 passes + loop)."""
    n, k, m = nkm
    rng = np.random.default_rng(n + k + m)
    w, deq = int4_weight(dev, "int4", n, k, torch.float16, 128, rng)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(dev)
    y = matmul_nt(x, w, dtype=torch.float32)
    assert O.max_rel_err(y.cpu().numpy(), x.float().cpu().numpy().astype(np.float64) @ deq.T) <= TOL


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
@pytest.mark.parametrize("sdt,bs", [(torch.float16, 32), (torch.bfloat16, 64), (torch.float32, 128), (None, 32)])
@pytest.mark.parametrize("m", [1, 5, 16])
def test_gemv_int4_mfma_parity(dev, fmt, sdt, bs, m):
    """INT4/UINT4 x fp16 GEMV on the f16-MFMA kernel (K a multiple of 128), ragged N."""
    n, k = 1000, 512
    rng = np.random.default_rng(m * 11 + bs)
    w, deq = int4_weight(dev, fmt, n, k, sdt, bs, rng)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(dev)
    y = matmul_nt(x, w, dtype=torch.float32)
    assert O.max_rel_err(y.cpu().numpy(), x.float().cpu().numpy().astype(np.float64) @ deq.T) <= TOL


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
@pytest.mark.parametrize("sdt,bs", [(torch.float16, 32), (torch.bfloat16, 64), (torch.float32, 32),
                                    (torch.float16, 128), (None, 32)])
@pytest.mark.parametrize("nkm", [(1000, 1024, 2), (6144, 4096, 8), (300, 2048, 16), (4100, 2048, 5),
                                 (14336, 1024, 3), (300, 3072, 16)])
def test_gemv_int4_xr_parity(dev, fmt, sdt, bs, nkm):
    """INT4/UINT4 x fp16 GEMV with the activations in registers (K = 1024, 2048, 4096 and
    2 <= M <= 16): 1 row tile per workgroup (1000, 300 rows: 4- and 8-row workgroups), 2 (6144,
    4100 rows: 24 and 20) and 4 (14336 rows: 56), every scale type and group size, one, two and
    four K super-steps per wave.  K = 3072 (slices of 6-48 scale bytes) takes the LDS-staging
    kernel."""
    n, k, m = nkm
    rng = np.random.default_rng(n + k + m + bs)
    w, deq = int4_weight(dev, fmt, n, k, sdt, bs, rng)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(dev)
    y = matmul_nt(x, w, dtype=torch.float32)
    assert O.max_rel_err(y.cpu().numpy(), x.float().cpu().numpy().astype(np.float64) @ deq.T) <= TOL


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
@pytest.mark.parametrize("bs", [32, 128])
def test_gemv_int4_xr_one_hot_is_exact(dev, fmt, bs):
    """Register-activation INT4 GEMV (6144 x 4096, M = 8: two row tiles per workgroup, four
    super-steps per wave): one-hot rows recover code * scale exactly for columns in every
    wave's K slice, block, lane group and code position."""
    n, k, m = 6144, 4096, 8
    rng = np.random.default_rng(40 + bs)
    w, deq = int4_weight(dev, fmt, n, k, torch.float16, bs, rng)
    for cols in ([0, 1, 7, 8, 31, 32, 127, 128], [511, 512, 1000, 2047, 2048, 3000, 4094, 4095]):
        x = torch.zeros((m, k), dtype=torch.float16, device=dev)
        x[torch.arange(m), torch.tensor(cols)] = 1.0
        y = matmul_nt(x, w, dtype=torch.float32).cpu().numpy()
        assert np.array_equal(y, deq[:, cols].T.astype(np.float32)), cols


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
def test_gemv_int4_one_hot_is_exact(dev, fmt):
    """One-hot fp16 activation rows recover code * scale exactly (fp32 out): nibble order,
    block K order and the per-block scale FMA line up."""
    n, k, m = 512, 1024, 16
    rng = np.random.default_rng(12)
    w, deq = int4_weight(dev, fmt, n, k, torch.float16, 32, rng)
    cols = rng.choice(k, m, replace=False)
    x = torch.zeros((m, k), dtype=torch.float16, device=dev)
    x[torch.arange(m), torch.from_numpy(cols)] = 1.0
    y = matmul_nt(x, w, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(y, deq[:, cols].T.astype(np.float32))


def test_gemv_int4_14336x4096_shape(dev):
    """INT4 g32 fp16-scale GEMV at 14336 x 4096, fp16 x [1, 4096] -> fp16."""
    n, k = 14336, 4096
    rng = np.random.default_rng(6)
    w, deq = int4_weight(dev, "int4", n, k, torch.float16, 32, rng)
    x = torch.from_numpy(rng.standard_normal((1, k)).astype(np.float16)).to(dev)
    y = matvec(w, x[0], output_dtype=torch.float16)
    ref = deq @ x[0].float().cpu().numpy().astype(np.float64)
    assert O.max_rel_err(y.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "int4", "uint4"])
@pytest.mark.parametrize("k", [2048, 4096, 8192, 14336, 16384])
def test_gemv_rows_one_hot_is_exact(dev, fmt, k):
    """M = 1 row-streaming kernels (K a multiple of 2048): one-hot activations recover
    deq(W)[:, j] exactly for columns across lanes, half-rows and code positions."""
    n = 200  # ragged: 200 rows = 6.25 workgroups of 32
    rng = np.random.default_rng(k)
    if fmt == "fp4_e2m1":
        w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
        xdt = torch.bfloat16
    else:
        w, deq = int4_weight(dev, fmt, n, k, torch.float16, 32, rng)
        xdt = torch.float16
    for j in [0, 1, 2, 3, 5, 7, 8, 31, 32, 33, 1000, 2047, 2048, 10241, k - 1]:
        if j >= k:
            continue
        x = torch.zeros(k, dtype=xdt, device=dev)
        x[j] = 1.0
        y = matvec(w, x, torch.float32).cpu().numpy()
        assert np.array_equal(y, deq[:, j].astype(np.float32)), f"column {j}"


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
@pytest.mark.parametrize("sdt,bs", [(torch.float16, 32), (torch.bfloat16, 64), (torch.float32, 128), (None, 32)])
@pytest.mark.parametrize("nk", [(1000, 4096), (300, 2048), (64, 8192)])
def test_gemv_rows_int4_parity(dev, fmt, sdt, bs, nk):
    """M = 1 INT4/UINT4 x fp16 on the row-streaming kernel, every scale dtype and group size."""
    n, k = nk
    rng = np.random.default_rng(n + k + bs)
    w, deq = int4_weight(dev, fmt, n, k, sdt, bs, rng)
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float16)).to(dev)
    y = matvec(w, x, torch.float32)
    assert O.max_rel_err(y.cpu().numpy(), deq @ x.float().cpu().numpy().astype(np.float64)) <= TOL


@pytest.mark.parametrize("nk", [(4096, 14336), (200, 10240), (333, 16384)])
def test_gemv_rows_fp4_long_rows_parity(dev, nk):
    """M = 1 FP4 rows kernel with 4 rows per wave (K of 10240 .. 16384, e.g. the SwiGLU down
    projection 4096 x 14336), ragged N."""
    n, k = nk
    rng = np.random.default_rng(n + k)
    w, deq = make_weight(dev, "fp4_e2m1", n, k, "e8m0", rng)
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(dev).to(torch.bfloat16)
    y = matvec(w, x, torch.float32)
    assert O.max_rel_err(y.cpu().numpy(), deq @ bf16_np(x).astype(np.float64)) <= TOL


def test_matvec_thread_true_uses_native_gemv(dev):
    rng = np.random.default_rng(1)
    w, deq = make_weight(dev, "fp4_e2m1", 128, 256, "e8m0", rng)
    v = torch.from_numpy(rng.standard_normal(256).astype(np.float32)).to(dev).to(torch.bfloat16)
    y = matvec(w, v, torch.float32, thread=True)
    assert O.max_rel_err(y.cpu().numpy(), deq @ bf16_np(v).astype(np.float64)) <= TOL


# ----------------------------------------------------------------------------- GEMM paths
@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
def test_gemm_weight_parity(dev, fmt):
    """Prefill-shaped (M > 16) packed-weight GEMM, C = A @ deq(W)^T."""
    m, n, k = 96, 160, 256
    rng = np.random.default_rng(21)
    w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    c = matmul_nt(a, w, dtype=torch.bfloat16)
    assert O.max_rel_err(bf16_np(c), O.matmul_reference(bf16_np(a), deq.T)) <= TOL


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
@pytest.mark.parametrize("mnk", [(128, 256, 128), (200, 300, 256), (33, 1000, 512), (513, 257, 384)])
@pytest.mark.parametrize("cdt", [torch.bfloat16, torch.float32])
def test_gemm_w_tiles_and_tails(dev, fmt, mnk, cdt):
    """Family 2 dequant-to-bf16 MFMA GEMM (the explicit scope requires the native kernel):
    whole and ragged 128 x 256 tiles, E8M0 block scales."""
    m, n, k = mnk
    rng = np.random.default_rng(m + 3 * n + k)
    w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    c = matmul_nt(a, w, scope="ThreadGroup", dtype=cdt)
    assert c.dtype is cdt and c.shape == (m, n)
    assert O.max_rel_err(c.float().cpu().numpy(), bf16_np(a) @ deq.T) <= TOL


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
def test_gemm_w_unscaled_and_strided_activations(dev, fmt):
    m, n, k = 150, 270, 256
    rng = np.random.default_rng(31)
    w, deq = make_weight(dev, fmt, n, k, "none", rng)
    big = torch.from_numpy(rng.standard_normal((m, k + 64)).astype(np.float32)).to(dev).to(torch.bfloat16)
    a = big[:, 32:32 + k]  # row stride k + 64 elements, 64-byte offset
    c = matmul_nt(a, w, scope="ThreadGroup", dtype=torch.float32)
    assert O.max_rel_err(c.cpu().numpy(), bf16_np(a) @ deq.T) <= TOL


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
def test_gemm_w_one_hot_is_exact(dev, fmt):
    """One-hot activation rows (1.0 at column j) recover deq(W)[:, j] exactly in fp32:
    code order, scale bytes and the MFMA's K order all line up."""
    m, n, k = 128, 256, 512
    rng = np.random.default_rng(9)
    w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
    cols = rng.choice(k, m, replace=True)
    a = torch.zeros((m, k), dtype=torch.bfloat16, device=dev)
    a[torch.arange(m), torch.from_numpy(cols)] = 1.0
    c = matmul_nt(a, w, scope="ThreadGroup", dtype=torch.float32).cpu().numpy()
    assert np.array_equal(c, deq[:, cols].T.astype(np.float32))


@pytest.mark.parametrize("fmt", ["fp6_e3m2", "fp6_e2m3"])
def test_gemm_w_fp6_2048x11008x4096_full_size_sampled(dev, fmt):
    """The FP6 prefill GEMM at full size: A bf16 [2048, 4096], W = MX-quantised N(0, 0.02) [11008, 4096]
    (block-32 E8M0); 64 x 512 sampled outputs against the fp64 oracle, which decodes the sampled W rows
    from the host copy of the packed bytes."""
    m, n, k = 2048, 11008, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    a = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
    w = quantize_mx(torch.randn((n, k), device=dev, generator=g) * 0.02, fmt)
    c = matmul_nt(a, w, scope="ThreadGroup", dtype=torch.bfloat16)
    rng = np.random.default_rng(5)
    rows, cols = stratified(rng, m, 1), stratified(rng, n, 1)  # one output in every 32 x 32 tile
    deq = host_dequant_rows(w, cols)
    ref = bf16_np(a)[rows] @ deq.T
    assert O.max_rel_err(bf16_np(c)[np.ix_(rows, cols)], ref) <= TOL


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
@pytest.mark.parametrize("sdt,bs", [(torch.float16, 128), (torch.float16, 32), (torch.bfloat16, 64), (torch.float32, 32),
                                    (None, 32)])
@pytest.mark.parametrize("mnk", [(128, 256, 128), (200, 300, 512), (513, 257, 384)])
def test_gemm_w_int4_tiles_and_groups(dev, fmt, sdt, bs, mnk):
    """INT4/UINT4 weights x fp16 activations on the f16-MFMA GEMM with per-group scales:
    whole and ragged tiles, groups of 32 / 64 / 128, every scale dtype, unscaled."""
    m, n, k = mnk
    rng = np.random.default_rng(m + n + k + bs)
    w, deq = int4_weight(dev, fmt, n, k, sdt, bs, rng)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(dev)
    c = matmul_nt(a, w, scope="ThreadGroup", dtype=torch.float32)
    assert c.shape == (m, n)
    assert O.max_rel_err(c.cpu().numpy(), a.float().cpu().numpy().astype(np.float64) @ deq.T) <= TOL


@pytest.mark.parametrize("fmt", ["int4", "uint4"])
@pytest.mark.parametrize("bs", [32, 128])
def test_gemm_w_int4_one_hot_is_exact(dev, fmt, bs):
    """One-hot fp16 activation rows recover code * scale exactly in fp32: nibble order, the
    MFMA K order and the per-group scale multiply all line up."""
    m, n, k = 256, 512, 512
    rng = np.random.default_rng(bs)
    w, deq = int4_weight(dev, fmt, n, k, torch.float16, bs, rng)
    cols = rng.choice(k, m, replace=True)
    a = torch.zeros((m, k), dtype=torch.float16, device=dev)
    a[torch.arange(m), torch.from_numpy(cols)] = 1.0
    c = matmul_nt(a, w, scope="ThreadGroup", dtype=torch.float32).cpu().numpy()
    assert np.array_equal(c, deq[:, cols].T.astype(np.float32))


def test_gemm_w_int4_prefill_shape(dev):
    """Attention-projection prefill shape: 512 tokens x fp16 [512, 4096] times INT4 g128
    fp16-scale weights [6144, 4096] (q, k and v rows stacked), fp16 out."""
    m, n, k = 512, 6144, 4096
    rng = np.random.default_rng(17)
    w, deq = int4_weight(dev, "int4", n, k, torch.float16, 128, rng)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(dev)
    c = matmul_nt(a, w, scope="ThreadGroup", dtype=torch.float16)
    rows, cols = stratified(rng, m, 4), stratified(rng, n, 1)  # outputs in every 32 x 32 tile
    ref = a.float().cpu().numpy().astype(np.float64)[rows] @ deq[cols].T
    assert O.max_rel_err(c.float().cpu().numpy()[np.ix_(rows, cols)], ref) <= TOL


def _gemm_w_call(name, a, w, c, *extra):
    from tinygrad_mi355x.runtime import kernels as K
    sdt = K.dtype_id(w.scales.dtype) if w.scales is not None else -1
    K.call(name, a.data_ptr(), K.dtype_id(a.dtype), a.shape[0], a.stride(0), w.data.data_ptr(), K.FORMAT_IDS[w.format],
           w.shape[0], w.shape[1], K.ptr(w.scales), sdt, w.block_size, c.data_ptr(), K.dtype_id(c.dtype), c.stride(0),
           *extra, torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("fmt,mnk,splits", [("fp4_e2m1", (512, 4096, 14336), 4), ("fp4_e2m1", (200, 1000, 1024), 3),
                                            ("fp6_e3m2", (300, 512, 640), 8), ("int4", (512, 6144, 4096), 2),
                                            ("int4", (129, 256, 1152), 5), ("fp4_e2m1", (64, 1002, 512), 4)])
def test_gemm_w_split_k(dev, fmt, mnk, splits):
    """Split-K (fp32 partials per K range, summed in a fixed order) against the single-pass
    GEMM and the fp64 oracle; two runs are bit-identical; a split count beyond the K steps, or
    N % 4 != 0 (the last case), falls back to the single pass exactly."""
    from tinygrad_mi355x.runtime import kernels as K
    m, n, k = mnk
    rng = np.random.default_rng(m + n + k)
    if fmt == "int4":
        w, deq = int4_weight(dev, fmt, n, k, torch.float16, 128, rng)
        a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(dev)
    else:
        w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
        a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    ws_bytes = K.load_library().tgm_gemm_w_split_workspace(m, n, splits)
    ws = torch.empty(max(ws_bytes // 4, 4), dtype=torch.float32, device=dev)
    one = torch.empty((m, n), dtype=torch.float32, device=dev)
    _gemm_w_call("tgm_gemm_w", a, w, one)
    runs = []
    for _ in range(2):
        c = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        _gemm_w_call("tgm_gemm_w_split", a, w, c, splits, ws.data_ptr(), ws_bytes)
        runs.append(c)
    assert torch.equal(runs[0], runs[1])
    if n % 4:
        assert torch.equal(runs[0], one)
    ref = a.float().cpu().numpy().astype(np.float64) @ deq.T
    # fp32 outputs: only summation order differs (K up to 14336 terms)
    assert O.max_rel_err(runs[0].cpu().numpy(), ref) <= 1e-3
    assert O.max_rel_err(runs[0].cpu().numpy(), one.cpu().numpy().astype(np.float64)) <= 1e-3


def test_gemm_w_split_k_rejects_a_small_workspace(dev):
    from tinygrad_mi355x.runtime import kernels as K
    rng = np.random.default_rng(2)
    w, _ = make_weight(dev, "fp4_e2m1", 256, 1024, "e8m0", rng)
    a = torch.zeros((128, 1024), dtype=torch.bfloat16, device=dev)
    c = torch.empty((128, 256), dtype=torch.float32, device=dev)
    ws = torch.empty(16, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="workspace"):
        _gemm_w_call("tgm_gemm_w_split", a, w, c, 4, ws.data_ptr(), 64)


@pytest.mark.parametrize("fa,fb", [("fp4_e2m1", "fp4_e2m1"), ("fp6_e2m3", "fp4_e2m1"), ("fp6_e3m2", "fp6_e2m3")])
def test_gemm_mx_parity(dev, fa, fb):
    m, n, k = 64, 96, 256
    rng = np.random.default_rng(23)
    a, deq_a = make_weight(dev, fa, m, k, "e8m0", rng)
    b, deq_b = make_weight(dev, fb, n, k, "e8m0", rng)
    c = matmul_nt(a, b, dtype=torch.float32)
    assert O.max_rel_err(c.cpu().numpy(), O.matmul_reference(deq_a, deq_b.T)) <= TOL


@pytest.mark.parametrize("mnk", [(256, 256, 256), (300, 520, 512), (1000, 777, 768), (40, 1100, 1024), (513, 33, 256)])
@pytest.mark.parametrize("cdt", [torch.bfloat16, torch.float16, torch.float32])
def test_gemm_mx_fp4_tiles_and_tails(dev, mnk, cdt):
    """FP4 x FP4 scaled-MFMA GEMM: whole and ragged 256 x 256 tiles, every output dtype."""
    m, n, k = mnk
    rng = np.random.default_rng(m * 7 + n + k)
    a, deq_a = make_weight(dev, "fp4_e2m1", m, k, "e8m0", rng)
    b, deq_b = make_weight(dev, "fp4_e2m1", n, k, "e8m0", rng)
    c = matmul_nt(a, b, dtype=cdt)
    assert c.dtype is cdt and c.shape == (m, n)
    assert O.max_rel_err(c.float().cpu().numpy(), deq_a @ deq_b.T) <= TOL


def test_gemm_mx_fp4_one_hot_is_exact(dev):
    """A row of one-hot FP4 codes (1.0 at column j) recovers deq(B)[:, j] exactly: scale
    bytes, nibble order and the MFMA's K order all line up."""
    m, n, k = 256, 256, 512
    rng = np.random.default_rng(8)
    b, deq_b = make_weight(dev, "fp4_e2m1", n, k, "e8m0", rng)
    cols = rng.choice(k, m, replace=True)
    codes = np.zeros((m, k), np.uint8)
    codes[np.arange(m), cols] = 2  # E2M1 code 2 = 1.0
    data = O.pack_codes(codes, 4)
    e = np.full((m, k // 32), 127, np.uint8)
    a = PackedTensor(torch.from_numpy(data).to(dev), "fp4_e2m1", (m, k),
                     torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu), 32)
    c = matmul_nt(a, b, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(c, deq_b[:, cols].T.astype(np.float32))


def test_gemm_mx_fp4_stream_one_hot_is_exact(dev):
    """The persistent FP4 x FP4 kernel (K a multiple of 1024, 289 tiles: workgroups walk two tiles)
    with one-hot A rows whose E8M0 scales vary per block: C is deq(B)[:, j] times A's scale of block
    j / 32, exactly, in every output element -- the scale byte of every block, A's and B's, reaches
    its MFMA (the per-half scale words and the byte each substep's MFMA selects)."""
    m, n, k = 4352, 4352, 1024
    rng = np.random.default_rng(12)
    b, deq_b = make_weight(dev, "fp4_e2m1", n, k, "e8m0", rng)
    cols = rng.choice(k, m, replace=True)
    codes = np.zeros((m, k), np.uint8)
    codes[np.arange(m), cols] = 2  # E2M1 code 2 = 1.0
    e = (127 + rng.integers(-3, 4, (m, k // 32))).astype(np.uint8)
    a = PackedTensor(torch.from_numpy(O.pack_codes(codes, 4)).to(dev), "fp4_e2m1", (m, k),
                     torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu), 32)
    c = matmul_nt(a, b, dtype=torch.float32).cpu().numpy()
    scale_a = np.exp2(e[np.arange(m), cols // 32].astype(np.float64) - 127)
    assert np.array_equal(c, (deq_b[:, cols].T * scale_a[:, None]).astype(np.float32))


@pytest.mark.parametrize("mnk", [(8192, 8192, 8192), (4096, 14336, 4096)])
def test_gemm_mx_fp4_full_size_sampled(dev, mnk):
    """The FP4 x FP4 GEMMs at full size (operands MX-quantised from N(0,1)) against the fp64 oracle,
    which decodes the sampled rows from the host copies of the packed bytes.  Rows are sampled one per
    32-row band and columns two per 32-column band, so every 32 x 32 MFMA tile of the output -- every
    workgroup and slot of the XCD-aware tile order -- has sampled outputs."""
    m, n, k = mnk
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    a = quantize_mx(torch.randn((m, k), device=dev, generator=g), "fp4_e2m1")
    b = quantize_mx(torch.randn((n, k), device=dev, generator=g), "fp4_e2m1")
    c = matmul_nt(a, b, dtype=torch.bfloat16)
    rng = np.random.default_rng(4)
    rows, cols = stratified(rng, m, 1), stratified(rng, n, 2)
    ref = host_dequant_rows(a, rows) @ host_dequant_rows(b, cols).T
    assert O.max_rel_err(bf16_np(c)[np.ix_(rows, cols)], ref) <= TOL


@pytest.mark.parametrize("mnk", [(2100, 1300, 1024), (4352, 4352, 2048), (8192, 8448, 1024)])
@pytest.mark.parametrize("cdt", [torch.bfloat16, torch.float16, torch.float32])
def test_gemm_mx_fp4_persistent_stream(dev, mnk, cdt):
    """FP4 x FP4 with K a multiple of 1024 runs the persistent kernel (one workgroup per CU walking
    several tiles as one stream of K steps).  The shapes give workgroups 1 to 5 tiles, ragged last
    tiles, tile counts that are and are not multiples of 8 (54, 289, 1056), and K = 1024, where a
    workgroup moves to its next tile every four steps; every 32 x 32 output tile is sampled."""
    m, n, k = mnk
    print(f"persistent FP4 GEMM {m}x{n}x{k} {cdt}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(m + n + k)
    a = quantize_mx(torch.randn((m, k), device=dev, generator=g), "fp4_e2m1")
    b = quantize_mx(torch.randn((n, k), device=dev, generator=g), "fp4_e2m1")
    c = matmul_nt(a, b, dtype=cdt)
    assert c.dtype is cdt and c.shape == (m, n)
    rng = np.random.default_rng(7)
    rows, cols = stratified(rng, m, 1), stratified(rng, n, 1)
    ref = host_dequant_rows(a, rows) @ host_dequant_rows(b, cols).T
    assert O.max_rel_err(c.float().cpu().numpy()[np.ix_(rows, cols)], ref) <= TOL


MX_PAIRS = [(fa, fb) for fa in ("fp4_e2m1", "fp6_e2m3", "fp6_e3m2") for fb in ("fp4_e2m1", "fp6_e2m3", "fp6_e3m2")]


@pytest.mark.parametrize("fa,fb", MX_PAIRS)
@pytest.mark.parametrize("scaled", [(True, True), (True, False), (False, True), (False, False)])
def test_gemm_mx_every_fp4_fp6_pair(dev, fa, fb, scaled):
    """Every FP4 / FP6 pair, each side E8M0 block-32 scaled or unscaled, on the native scaled MFMA
    (scope="Wave" raises instead of falling back): ragged 256 x 128 tiles, K = 640 (five steps,
    two scale batches)."""
    m, n, k = 300, 200, 640
    rng = np.random.default_rng(MX_PAIRS.index((fa, fb)) * 4 + 2 * scaled[0] + scaled[1])
    a, deq_a = make_weight(dev, fa, m, k, "e8m0" if scaled[0] else None, rng)
    b, deq_b = make_weight(dev, fb, n, k, "e8m0" if scaled[1] else None, rng)
    c = matmul_nt(a, b, scope="Wave", dtype=torch.float32)
    assert c.shape == (m, n)
    assert O.max_rel_err(c.cpu().numpy(), deq_a @ deq_b.T) <= TOL


@pytest.mark.parametrize("fa,fb", [("fp6_e2m3", "fp6_e3m2"), ("fp4_e2m1", "fp6_e3m2"), ("fp6_e3m2", "fp4_e2m1")])
def test_gemm_mx_unscaled_pair_is_exact(dev, fa, fb):
    """Two unscaled packed operands (the reference's FP8 intermediate, dx12.py:115-138) with one
    nonzero code per row of A: every output is one exact product, so the result is bit-exact."""
    m, n, k = 256, 128, 256
    rng = np.random.default_rng(5)
    b, deq_b = make_weight(dev, fb, n, k, None, rng)
    cols = rng.choice(k, m)
    bits = FORMATS[fa][0]
    codes = np.zeros((m, k), np.uint8)
    codes[np.arange(m), cols] = rng.integers(1, 1 << bits, m)
    a = PackedTensor(torch.from_numpy(O.pack_codes(codes, bits)).to(dev), fa, (m, k))
    deq_a = O.dequant_f64(O.pack_codes(codes, bits), fa, (m, k), None, 32)
    c = matmul_nt(a, b, scope="Wave")
    assert c.dtype is torch.float32
    assert np.array_equal(c.cpu().numpy(), (deq_a @ deq_b.T).astype(np.float32))


@pytest.mark.parametrize("mnk", [(128, 128, 128), (257, 130, 384), (1024, 1024, 1024)])
def test_gemm_mx_fp4_pairs_with_k_a_multiple_of_128(dev, mnk):
    """FP4 x FP4 with both scales and K not a multiple of 256 takes the general kernel."""
    m, n, k = mnk
    rng = np.random.default_rng(k)
    a, deq_a = make_weight(dev, "fp4_e2m1", m, k, "e8m0", rng)
    b, deq_b = make_weight(dev, "fp4_e2m1", n, k, "e8m0", rng)
    c = matmul_nt(a, b, scope="Wave", dtype=torch.bfloat16)
    assert O.max_rel_err(bf16_np(c), deq_a @ deq_b.T) <= TOL


def _fp8(dev, shape, dt, rng):
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * 4).to(dev)
    return x.to(dt)


@pytest.mark.parametrize("da,db", [(torch.float8_e4m3fn, torch.float8_e4m3fn), (torch.float8_e5m2, torch.float8_e5m2),
                                   (torch.float8_e4m3fn, torch.float8_e5m2)])
@pytest.mark.parametrize("mnk", [(300, 200, 640), (64, 1100, 128)])
def test_gemm_fp8_parity(dev, da, db, mnk):
    """Ordinary FP8 operands on the scaled MFMA with unit scales: matmul_nt binds both K-last;
    matmul stages a row-major right operand with tgm_transpose8."""
    m, n, k = mnk
    rng = np.random.default_rng(m + n + k)
    a, b = _fp8(dev, (m, k), da, rng), _fp8(dev, (n, k), db, rng)
    ref = a.float().cpu().numpy().astype(np.float64) @ b.float().cpu().numpy().astype(np.float64).T
    c = matmul_nt(a, b, scope="Wave")
    assert c.dtype is torch.float32 and O.max_rel_err(c.cpu().numpy(), ref) <= TOL
    rowmajor = torch.empty((k, n), dtype=db, device=dev)
    rowmajor.view(torch.uint8).copy_(b.view(torch.uint8).t())
    c2 = matmul(a, rowmajor, scope="Wave", dtype=torch.bfloat16)
    assert O.max_rel_err(bf16_np(c2), ref) <= TOL


def test_gemm_fp8_per_tensor_scales(dev):
    """Per-tensor fp32 factors (torch._scaled_mm's) multiply the fp32 sums before rounding."""
    rng = np.random.default_rng(3)
    a, b = _fp8(dev, (256, 256), torch.float8_e4m3fn, rng), _fp8(dev, (128, 256), torch.float8_e4m3fn, rng)
    sa, sb = torch.tensor(0.125, device=dev), torch.tensor(3.0, device=dev)
    c = linalg.dense_matmul_nt(a, b, torch.float32, sa, sb)
    ref = a.float().cpu().numpy().astype(np.float64) @ b.float().cpu().numpy().astype(np.float64).T * 0.375
    assert O.max_rel_err(c.cpu().numpy(), ref) <= TOL


def test_failures_are_cached_per_candidate(dev, monkeypatch):
    """A native rejection (an MX pair whose K is not a whole number of 32-element blocks: the
    block-scaled MFMA GEMM has no kernel for it) is cached under its exact candidate key: the
    first auto call tries the native kernel once and falls back, a repeat skips the native
    attempt, and an explicit scope re-raises the cached reason (linalg.py:188-198, :216-223)."""
    linalg.matrix_failures.clear()
    rng = np.random.default_rng(2)
    m, n, k = 64, 96, 48
    a, deq_a = make_weight(dev, "fp4_e2m1", m, k, "e8m0", rng)
    b, deq_b = make_weight(dev, "fp4_e2m1", n, k, "e8m0", rng)
    attempts = []
    native = linalg._mx_nt

    def counting(*args):
        attempts.append(args)
        return native(*args)

    monkeypatch.setattr(linalg, "_mx_nt", counting)
    ref = deq_a @ deq_b.T
    first = matmul_nt(a, b, dtype=torch.float32)
    assert len(attempts) == 1 and len(linalg.matrix_failures) == 1
    (key, reason), = linalg.matrix_failures.items()
    assert key[0] == "tgm_gemm_mx" and "tgm_gemm_mx" in reason
    second = matmul_nt(a, b, dtype=torch.float32)
    assert len(attempts) == 1  # the cached rejection skips the native kernel
    # the fallback decodes both operands and runs the exact-width GEMM: exact here
    assert np.array_equal(first.cpu().numpy(), ref.astype(np.float32))
    assert torch.equal(first, second)
    with pytest.raises(RuntimeError, match="candidate rejected"):
        matmul_nt(a, b, scope="Wave", dtype=torch.float32)
    assert len(attempts) == 1
    linalg.matrix_failures.clear()


def test_fp64_operands_choose_no_native_kernel(dev):
    """fp64 activations have no native family: auto computes exactly at fp64, nothing is cached."""
    linalg.matrix_failures.clear()
    rng = np.random.default_rng(2)
    w, deq = make_weight(dev, "int4", 32, 64, "none", rng)
    x = torch.ones((2, 64), dtype=torch.float64, device=dev)
    out = matmul_nt(x, w)
    assert out.dtype is torch.float64 and not linalg.matrix_failures
    assert np.array_equal(out.cpu().numpy(), np.ones((2, 64)) @ deq.T)


def test_transpose16_honours_the_column_stride_of_a_single_row(dev):
    """A single-row view read at every other column (base[0:1, ::2], the right operand of a
    K = 1 product) is staged with its column stride; so are multi-row strided views."""
    base = torch.arange(64, dtype=torch.float32, device=dev).reshape(2, 32).to(torch.bfloat16)
    for view in (base[0:1, ::2], base[:, ::2], base[:, 1::4], base[0:1, :]):
        assert torch.equal(linalg.transpose16(view), view.t().contiguous()), view.stride()
    b = base[0:1, ::2]
    a = torch.arange(1, 33, dtype=torch.float32, device=dev).reshape(32, 1).to(torch.bfloat16)
    c = matmul(a, b, dtype=torch.float32)
    assert torch.equal(c.cpu(), a.float().cpu() @ b.float().cpu())


def test_concurrent_callers_get_their_sequential_results(dev):
    """Packed products issued from 6 threads at once (GEMV and GEMM families, several formats)
    equal the same products issued one after another, bit for bit."""
    from concurrent.futures import ThreadPoolExecutor
    from threading import Barrier

    rng = np.random.default_rng(44)
    cases = []
    for i, (fmt, m, n, k) in enumerate([("fp4_e2m1", 1, 512, 2048), ("fp6_e2m3", 40, 256, 256),
                                        ("fp4_e2m1", 4, 1024, 512), ("fp6_e3m2", 1, 300, 256),
                                        ("fp4_e2m1", 200, 512, 512), ("fp6_e2m3", 8, 128, 384)]):
        w, _ = make_weight(dev, fmt, n, k, "e8m0", rng)
        a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
        cases.append((a, w))
    expected = [matmul_nt(a, w, dtype=torch.float32) for a, w in cases]
    torch.cuda.synchronize()
    barrier = Barrier(len(cases))

    def run(i: int) -> torch.Tensor:
        barrier.wait()
        out = [matmul_nt(cases[i][0], cases[i][1], dtype=torch.float32) for _ in range(5)]
        torch.cuda.synchronize()
        return out

    with ThreadPoolExecutor(max_workers=len(cases)) as workers:
        results = list(workers.map(run, range(len(cases))))
    for got, want in zip(results, expected):
        assert all(torch.equal(g, want) for g in got)



# At least one round of 128 x 256 tiles (256 CUs) with K a multiple of 512 runs the persistent weight
# GEMM (gemm_w_stream): 1000 x 8200 is 8 x 33 = 264 tiles, so some workgroups take two tiles.
@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e2m3", "fp6_e3m2"])
@pytest.mark.parametrize("scale_kind", ["e8m0", "none"])
def test_gemm_w_stream_one_hot_is_exact(dev, fmt, scale_kind):
    """One-hot activation rows recover deq(W)[:, j] exactly (fp32 and bf16 outputs) in every tile of the
    persistent kernel, ragged edges included: code order, the two MX blocks a lane decodes per step,
    their scale bytes, the MFMA K order, the tile walk and the epilogue all line up."""
    m, n, k = 1000, 8200, 512
    rng = np.random.default_rng(17)
    w, deq = make_weight(dev, fmt, n, k, scale_kind, rng)
    cols = rng.choice(k, m, replace=True)
    a = torch.zeros((m, k), dtype=torch.bfloat16, device=dev)
    a[torch.arange(m), torch.from_numpy(cols)] = 1.0
    want = deq[:, cols].T.astype(np.float32)
    for cdt in (torch.float32, torch.bfloat16):
        c = matmul_nt(a, w, scope="ThreadGroup", dtype=cdt).float().cpu().numpy()
        assert np.array_equal(c, want), cdt


@pytest.mark.parametrize("fmt", ["fp4_e2m1", "fp6_e3m2"])
def test_gemm_w_stream_parity(dev, fmt):
    """Random bf16 activations (a strided view) against the fp64 oracle on rows sampled in every
    32-row band, three output dtypes, K = 1024 (two scale batches per tile)."""
    m, n, k = 1000, 8200, 1024
    rng = np.random.default_rng(23)
    w, deq = make_weight(dev, fmt, n, k, "e8m0", rng)
    big = torch.from_numpy(rng.standard_normal((m, k + 64)).astype(np.float32)).to(dev).to(torch.bfloat16)
    a = big[:, 32:32 + k]
    rows = stratified(rng, m, 2)
    ref = bf16_np(a)[rows].astype(np.float64) @ deq.T
    for cdt in (torch.float32, torch.bfloat16, torch.float16):
        c = matmul_nt(a, w, scope="ThreadGroup", dtype=cdt)
        assert O.max_rel_err(bf16_np(c)[rows], ref) <= TOL, cdt
