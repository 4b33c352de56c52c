"""The allocation-free split-K GEMM (tgm_gemm_w_split_noalloc) against tgm_gemm_w_split.

Both run the same split-K kernels and the same fixed-order reduction; the only difference is
where the fp32 partials live (the library's static per-device array instead of a caller
workspace), so the outputs must be bit-identical.  Two calls in a row, the second smaller than
the first, check that a call never reads what an earlier call left in the shared array.
"""

import numpy as np
import pytest
import torch

import packed_oracle as O
from tinygrad_mi355x.codegen.decomp.mi355x import FORMATS, PackedTensor
from tinygrad_mi355x.runtime import kernels as K

pytestmark = pytest.mark.gpu


def _weight(dev, fmt, n, k, rng):
    bits = FORMATS[fmt][0]
    codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint8)
    data = torch.from_numpy(O.pack_codes(codes, bits)).to(dev)
    if fmt in ("int4", "uint4"):
        s_np = rng.uniform(0.005, 0.02, (n, k // 128)).astype(np.float16)
        return PackedTensor(data, fmt, (n, k), torch.from_numpy(s_np).to(dev), 128)
    e = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.uint8)
    return PackedTensor(data, fmt, (n, k), torch.from_numpy(e).to(dev).view(torch.float8_e8m0fnu), 32)


def _args(a, w, c):
    sdt = K.dtype_id(w.scales.dtype)
    return (a.data_ptr(), K.dtype_id(a.dtype), a.shape[0], a.stride(0), w.data.data_ptr(), K.FORMAT_IDS[w.format],
            w.shape[0], w.shape[1], w.scales.data_ptr(), sdt, w.block_size, c.data_ptr(), K.dtype_id(c.dtype),
            c.stride(0))


# (format, (M, N, K), splits): the 512-token down projection (4 x 512 x 4096 fp32 partials: exactly
# the 32 MiB capacity), then a smaller INT4 product with a ragged tile and five splits
CASES = [("fp4_e2m1", (512, 4096, 14336), 4), ("int4", (129, 256, 1152), 5)]


def test_noalloc_split_k_equals_the_workspace_form_on_consecutive_calls(dev):
    lib = K.load_library()
    capacity = lib.tgm_gemm_w_split_noalloc_capacity()
    assert capacity == 32 << 20
    stream = torch.cuda.current_stream().cuda_stream
    for fmt, (m, n, k), splits in CASES:
        print(f"noalloc split-K {fmt} M={m} N={n} K={k} splits={splits}", flush=True)
        rng = np.random.default_rng(m + n + k)
        w = _weight(dev, fmt, n, k, rng)
        adt = np.float16 if fmt == "int4" else np.float32
        a = torch.from_numpy(rng.standard_normal((m, k)).astype(adt)).to(dev)
        if fmt != "int4":
            a = a.to(torch.bfloat16)
        ws_bytes = lib.tgm_gemm_w_split_workspace(m, n, splits)
        assert 0 < ws_bytes <= capacity
        ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=dev)
        want = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        K.call("tgm_gemm_w_split", *_args(a, w, want), splits, ws.data_ptr(), ws_bytes, stream)
        got = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
        K.call("tgm_gemm_w_split_noalloc", *_args(a, w, got), splits, stream)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{fmt} {m}x{n}x{k}"
        deq = O.dequant_f64(w.data.cpu().numpy(), fmt, (n, k), w.scales.float().cpu().numpy(), w.block_size)
        rows = np.random.default_rng(1).choice(m, min(m, 32), replace=False)
        ref = a.float().cpu().numpy().astype(np.float64)[rows] @ deq.T
        assert O.max_rel_err(got.cpu().numpy()[rows], ref) <= 1e-3


def test_noalloc_split_k_rejects_partials_beyond_the_capacity(dev):
    rng = np.random.default_rng(3)
    w = _weight(dev, "fp4_e2m1", 4096, 4096, rng)
    a = torch.zeros((1024, 4096), dtype=torch.bfloat16, device=dev)
    c = torch.empty((1024, 4096), dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="static scratch"):
        K.call("tgm_gemm_w_split_noalloc", *_args(a, w, c), 4, torch.cuda.current_stream().cuda_stream)


def test_noalloc_split_k_on_the_null_stream_and_a_side_stream(dev):
    """The scratch address is looked up for the device the stream launches on: the null stream (the
    current device's) and a second stream of the current device give the workspace form's bits."""
    lib = K.load_library()
    rng = np.random.default_rng(11)
    m, n, k, splits = 64, 512, 2048, 4
    w = _weight(dev, "fp4_e2m1", n, k, rng)
    a = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(torch.bfloat16)
    ws_bytes = lib.tgm_gemm_w_split_workspace(m, n, splits)
    ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=dev)
    want = torch.empty((m, n), dtype=torch.float32, device=dev)
    K.call("tgm_gemm_w_split", *_args(a, w, want), splits, ws.data_ptr(), ws_bytes,
           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    print("noalloc split-K on the null stream", flush=True)
    got = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    K.call("tgm_gemm_w_split_noalloc", *_args(a, w, got), splits, None)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    print("noalloc split-K on a side stream", flush=True)
    side = torch.cuda.Stream(device=dev)
    got2 = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    K.call("tgm_gemm_w_split_noalloc", *_args(a, w, got2), splits, side.cuda_stream)
    side.synchronize()
    assert torch.equal(got2, want)
