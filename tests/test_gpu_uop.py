"""UOp kernels rendered to HIP and run on gfx950, and scheduled products on the MFMA GEMMs.

Rendered kernels are checked against numpy computing the same operations in the same dtypes
(bit-exact for integer, bool, f16, f32, f64 and bf16 arithmetic, where bf16 is fp32 arithmetic
rounded to bf16 after each operation; the device math library's EXP2 / LOG2 / SIN within 4 ulp
of fp32).  Scheduled matrix products -- lowered to the GEMMs or left as rendered kernels -- are
checked against the fp64 product of the same operands with the packed-product tolerance (max
relative error <= 1e-2; fp32 outputs within 1e-3).
"""

import numpy as np
import pytest

import packed_oracle as O
from tinygrad_mi355x.codegen.uop_matmul import lower_matmul
from tinygrad_mi355x.runtime import ops_mi355x as R
from tinygrad_mi355x.runtime.schedule import LinearGraph, compile_kernel, run_linear
from tinygrad_mi355x.uop.ops import AxisType, KernelInfo, Ops, UOp, dtypes

pytestmark = pytest.mark.gpu
DEV = "MI355X"
NP = {"bool": np.uint8, "int8": np.int8, "uint8": np.uint8, "int16": np.int16, "uint16": np.uint16,
      "int32": np.int32, "uint32": np.uint32, "int64": np.int64, "uint64": np.uint64, "float16": np.float16,
      "bfloat16": np.uint16, "float32": np.float32, "float64": np.float64, "float8_e4m3fn": np.uint8,
      "float8_e5m2": np.uint8}


@pytest.fixture(scope="module")
def device():
    d = R.get_device(DEV)
    yield d
    d.synchronize()


def run_sink(dev, sink, inputs: dict, var_vals=None, lower=False, input_slots=()):
    """Run one kernel (or, with ``lower``, its matmul lowering) on fresh buffers: ``inputs`` maps
    PARAM slots to arrays; returns every slot's contents afterwards."""
    params = sorted((u for u in sink.toposort() if u.op is Ops.PARAM), key=lambda u: u.arg.slot)
    by_slot = {p.arg.slot: p for p in params}
    # one CALL argument per slot up to the highest; slots the kernel does not read get a stand-in
    bufs = [UOp.new_buffer(DEV, by_slot[s].max_numel(), by_slot[s].dtype) if s in by_slot else
            UOp.new_buffer(DEV, 1, dtypes.uint8) for s in range(params[-1].arg.slot + 1)]
    bound = {}
    for p in params:
        b = bufs[p.arg.slot]
        if p.arg.slot in inputs:
            arr = np.ascontiguousarray(inputs[p.arg.slot])
            assert arr.nbytes == p.max_numel() * p.dtype.itemsize
            buf = dev.allocator.alloc(arr.nbytes)
            dev.allocator._copyin(buf, memoryview(arr.reshape(-1)).cast("B"))
            bound[b] = buf
    linear = UOp.linear(UOp.call(sink, *bufs))
    if lower:
        linear = lower_matmul(linear, tuple(bufs[s] for s in input_slots))
    done = run_linear(dev, linear, bound, var_vals, wait=True)
    out = {}
    for p in params:
        arr = np.empty(p.max_numel(), NP[p.dtype.name])
        dev.allocator._copyout(memoryview(arr).cast("B"), done[bufs[p.arg.slot]])
        out[p.arg.slot] = arr
    return out, linear


def elementwise(dt, fn, n, out_dt=None, name="ew"):
    a, b = UOp.param(1, dt, n, DEV), UOp.param(2, dt, n, DEV)
    o = UOp.param(0, out_dt or dt, n, DEV)
    i = UOp.range(n, 0)
    return o.index(i).store(fn(a.index(i), b.index(i))).end(i).sink(arg=KernelInfo(name=name))


# ----------------------------------------------------------------------------- elementwise
INT_DTYPES = [dtypes.int8, dtypes.uint8, dtypes.int16, dtypes.uint16, dtypes.int32, dtypes.uint32, dtypes.int64,
              dtypes.uint64]


@pytest.mark.parametrize("dt", INT_DTYPES, ids=lambda d: d.name)
def test_integer_arithmetic_wraps_to_its_width(device, dt):
    rng = np.random.default_rng(1)
    n = 1000  # not a multiple of the workgroup: the tail is guarded
    info = np.iinfo(NP[dt.name])
    a = rng.integers(info.min, info.max, n, dtype=NP[dt.name], endpoint=True)
    b = rng.integers(info.min, info.max, n, dtype=NP[dt.name], endpoint=True)
    sh = UOp.const(dt, 3)
    sink = elementwise(dt, lambda x, y: ((x * y + x - y) ^ (x << sh)).maximum(y >> sh) | (x & y), n, name=f"i_{dt.name}")
    out, _ = run_sink(device, sink, {1: a, 2: b})
    with np.errstate(over="ignore"):
        s = NP[dt.name](3)
        want = np.maximum((a * b + a - b) ^ (a << s), b >> s) | (a & b)
    np.testing.assert_array_equal(out[0], want)


def test_integer_division_truncates(device):
    rng = np.random.default_rng(2)
    n = 512
    a = rng.integers(-1000, 1000, n).astype(np.int32)
    b = rng.integers(1, 50, n).astype(np.int32) * rng.choice([-1, 1], n).astype(np.int32)
    out, _ = run_sink(device, elementwise(dtypes.int32, lambda x, y: x // y * 1000 + x % y, n, name="idiv"),
                      {1: a, 2: b})
    q = np.fix(a / b).astype(np.int32)
    np.testing.assert_array_equal(out[0], q * 1000 + (a - q * b))


@pytest.mark.parametrize("dt", [dtypes.float16, dtypes.float32, dtypes.float64], ids=lambda d: d.name)
def test_float_arithmetic_rounds_each_operation(device, dt):
    rng = np.random.default_rng(3)
    n = 4096
    t = NP[dt.name]
    a = rng.standard_normal(n).astype(t)
    b = (rng.standard_normal(n) + 3).astype(t)
    sink = elementwise(dt, lambda x, y: (x * y + x) / y - x.maximum(y) * UOp.const(dt, -0.0), n, name=f"f_{dt.name}")
    out, _ = run_sink(device, sink, {1: a, 2: b})
    want = ((a * b + a) / b - np.maximum(a, b) * t(-0.0)).astype(t)
    np.testing.assert_array_equal(out[0].view(NP[dt.name]), want)


def bf16(x):
    return O.bf16_to_f32(O.bf16_round(np.asarray(x, np.float32)))


def test_bfloat16_is_fp32_arithmetic_rounded_per_operation(device):
    rng = np.random.default_rng(4)
    n = 4096
    af, bf = bf16(rng.standard_normal(n)), bf16(rng.standard_normal(n) + 2)
    a, b = O.bf16_round(af), O.bf16_round(bf)
    out, _ = run_sink(device, elementwise(dtypes.bfloat16, lambda x, y: (x * y + x).maximum(y) / y, n, name="bf"),
                      {1: a, 2: b})
    want = bf16(bf16(np.maximum(bf16(bf16(af * bf) + af), bf)) / bf)
    np.testing.assert_array_equal(O.bf16_to_f32(out[0]), want)


def test_casts_and_bitcasts(device):
    rng = np.random.default_rng(5)
    n = 2048
    x = (rng.standard_normal(n) * 100).astype(np.float32)
    x[:4] = [0.5, -0.0, 255.0, 1e30]
    f32 = dtypes.float32
    i = UOp.range(n, 0)
    v = UOp.param(1, f32, n, DEV).index(i)
    in_range = (v < UOp.const(f32, 1e9)).alu(Ops.AND, UOp.const(f32, -1e9) < v)
    items = [UOp.param(0, dtypes.bfloat16, n, DEV).index(i).store(v.cast(dtypes.bfloat16)),
             UOp.param(2, dtypes.float16, n, DEV).index(i).store(v.cast(dtypes.float16)),
             UOp.param(3, dtypes.int32, n, DEV).index(i).store(in_range.where(v, 0.0).cast(dtypes.int32)),
             UOp.param(4, dtypes.bool, n, DEV).index(i).store(v.cast(dtypes.bool)),
             UOp.param(5, dtypes.int32, n, DEV).index(i).store(v.bitcast(dtypes.int32)),
             UOp.param(6, dtypes.float64, n, DEV).index(i).store(v.cast(dtypes.float64))]
    sink = UOp(Ops.SINK, None, tuple(it.end(i) for it in items), KernelInfo(name="casts"))
    out, _ = run_sink(device, sink, {1: x})
    np.testing.assert_array_equal(out[0], O.bf16_round(x))
    np.testing.assert_array_equal(out[2], x.astype(np.float16))
    np.testing.assert_array_equal(out[3], np.trunc(np.where(np.abs(x) < 1e9, x, 0)).astype(np.int32))
    np.testing.assert_array_equal(out[4], (x != 0).astype(np.uint8))
    np.testing.assert_array_equal(out[5], x.view(np.int32))
    np.testing.assert_array_equal(out[6], x.astype(np.float64))


def test_transcendentals_and_correctly_rounded_ops(device):
    rng = np.random.default_rng(6)
    n = 4096
    a = (rng.random(n) * 8 + 0.01).astype(np.float32)
    b = (rng.standard_normal(n) * 4).astype(np.float32)
    out_exact, _ = run_sink(device, elementwise(dtypes.float32, lambda x, y: x.sqrt() + x.reciprocal(), n,
                                                name="exact"), {1: a, 2: b})
    np.testing.assert_array_equal(out_exact[0], np.sqrt(a) + np.float32(1) / a)
    for fn, ref in ((lambda x, y: y.exp2(), np.exp2), (lambda x, y: x.log2(), None), (lambda x, y: y.sin(), np.sin)):
        out, _ = run_sink(device, elementwise(dtypes.float32, fn, n, name="tr"), {1: a, 2: b})
        want = (np.log2(a.astype(np.float64)) if ref is None else ref(b.astype(np.float64)))
        ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(out[0] - want) <= 4 * ulp + 1e-6)


def test_bool_and_fp8_loads(device):
    n = 256
    codes = np.arange(n, dtype=np.uint8)
    for dt, target in ((dtypes.fp8e4m3, "fp8e4m3"), (dtypes.fp8e5m2, "fp8e5m2")):
        sink = elementwise(dt, lambda x, y: x.cast(dtypes.float32) + y.cast(dtypes.float32), n, dtypes.float32,
                           name=f"fp8_{target}")
        out, _ = run_sink(device, sink, {1: codes, 2: np.zeros(n, np.uint8)})
        want = O.fp8_decode(codes, target)
        np.testing.assert_array_equal(out[0], want)  # NaN positions compare equal
    rng = np.random.default_rng(7)
    a, b = rng.integers(0, 3, n).astype(np.uint8), rng.integers(0, 2, n).astype(np.uint8)  # bytes 2 read as true
    out, _ = run_sink(device, elementwise(dtypes.bool, lambda x, y: x.ne(y), n, dtypes.bool, name="bools"), {1: a, 2: b})
    np.testing.assert_array_equal(out[0], ((a != 0) != (b != 0)).astype(np.uint8))


# ----------------------------------------------------------------------------- reductions
def test_reductions_gates_and_variables(device):
    rows, pad, cols = 300, 40, 48
    x, s, o = UOp.param(1, dtypes.float32, rows * pad, DEV), UOp.param(2, dtypes.float32, rows, DEV), \
        UOp.param(0, dtypes.float32, rows, DEV)
    r, c = UOp.range(rows, 0), UOp.range(cols, 1, AxisType.REDUCE)
    j = UOp.range(UOp.variable("n", 1, pad), 2, AxisType.REDUCE)
    total = (x.index(r * pad + c, c < pad) * s.index(r)).reduce(c, arg=Ops.ADD)
    peak = x.index(r * pad + j).reduce(j, arg=Ops.MAX)
    sink = o.index(r).store(total + peak).end(r).sink(arg=KernelInfo(name="rows"))
    rng = np.random.default_rng(8)
    xs = rng.integers(-50, 50, rows * pad).astype(np.float32)   # integer-valued: sums are exact
    sc = rng.integers(1, 4, rows).astype(np.float32)
    for nv in (1, 17, pad):
        out, _ = run_sink(device, sink, {1: xs, 2: sc}, {"n": nv})
        xm = xs.reshape(rows, pad)
        np.testing.assert_array_equal(out[0], xm.sum(1) * sc + xm[:, :nv].max(1))


def test_a_tinygrad_style_listing_with_lds_and_a_barrier(device):
    """A hand-written listing (the form tinygrad's codegen hands a renderer): each workgroup
    reverses its 256 values through LDS."""
    groups, local = 4, 256
    f32 = dtypes.float32
    out_p, in_p = UOp.param(0, f32, groups * local), UOp.param(1, f32, groups * local)
    g = UOp(Ops.SPECIAL, dtypes.int32, (UOp.const(dtypes.int32, groups),), "gidx0")
    lid = UOp(Ops.SPECIAL, dtypes.int32, (UOp.const(dtypes.int32, local),), "lidx0")
    lds = UOp(Ops.DEFINE_LOCAL, f32, (), (local, 0))
    gi = UOp(Ops.ADD, dtypes.int32, (UOp(Ops.MUL, dtypes.int32, (g, UOp.const(dtypes.int32, local))), lid))
    src_idx = UOp(Ops.INDEX, f32, (in_p, gi))
    v = UOp(Ops.LOAD, f32, (src_idx,))
    lds_w = UOp(Ops.INDEX, f32, (lds, lid))
    st1 = UOp(Ops.STORE, None, (lds_w, v))
    bar = UOp(Ops.BARRIER, None, (st1,))
    rev = UOp(Ops.SUB, dtypes.int32, (UOp.const(dtypes.int32, local - 1), lid))
    lds_r = UOp(Ops.INDEX, f32, (lds, rev))
    w = UOp(Ops.LOAD, f32, (lds_r, ), 1)
    dst = UOp(Ops.INDEX, f32, (out_p, gi))
    st2 = UOp(Ops.STORE, None, (dst, w))
    listing = [out_p, in_p, g, lid, lds, gi.src[0], gi, src_idx, v, lds_w, st1, bar, rev, lds_r, w, dst, st2]
    src = device.renderer.render(listing)
    assert "__shared__" in src and "__syncthreads();" in src
    prog = device.runtime("kernel", device.compiler.compile(src))
    x = np.arange(groups * local, dtype=np.float32)
    inb, outb = device.allocator.alloc(x.nbytes), device.allocator.alloc(x.nbytes)
    device.allocator._copyin(inb, memoryview(x).cast("B"))
    prog(outb, inb, global_size=(groups, 1, 1), local_size=(local, 1, 1), wait=True)
    got = np.empty_like(x)
    device.allocator._copyout(memoryview(got).cast("B"), outb)
    np.testing.assert_array_equal(got, x.reshape(groups, local)[:, ::-1].reshape(-1))


# ----------------------------------------------------------------------------- scheduled products
def matrix_sink(m, n, k, dtype, transposed=False, right_nk=False, activated=False, out_dtype=None):
    out_dtype = out_dtype or dtype
    output = UOp.param(0, out_dtype, m * n, DEV)
    left, right = UOp.param(1, dtype, m * k, DEV), UOp.param(2, dtype, k * n, DEV)
    row, col, inner = UOp.range(m, 1), UOp.range(n, 2), UOp.range(k, 0, AxisType.REDUCE)
    a = left.index(inner * m + row if transposed else row * k + inner)
    b = right.index(col * k + inner if right_nk else inner * n + col)
    product = a.cast(dtypes.float32) * b.cast(dtypes.float32)
    value = product.reduce(inner, arg=Ops.ADD)
    if activated:
        value = value.maximum(0.0)
    return output.index(row * n + col).store(value.cast(out_dtype)).end(row, col).sink(arg=KernelInfo(name="mm"))


def _operands(rng, m, n, k, dtype, transposed, right_nk):
    """Device bytes of A and B in the stored layouts, and their values as fp64 [m, k] / [k, n]."""
    if dtype == dtypes.bfloat16:
        av, bv = bf16(rng.standard_normal((m, k))), bf16(rng.standard_normal((k, n)))
        enc = O.bf16_round
    elif dtype == dtypes.float16:
        av, bv = rng.standard_normal((m, k)).astype(np.float16), rng.standard_normal((k, n)).astype(np.float16)
        enc = lambda v: v.astype(np.float16)  # noqa: E731
    else:
        codes = rng.integers(0, 256, (m * k + k * n)).astype(np.uint8)
        codes[(codes & 0x7F) == 0x7F] = 0x38  # no NaN codes
        av = O.fp8_decode(codes[:m * k], "fp8e4m3").reshape(m, k)
        bv = O.fp8_decode(codes[m * k:], "fp8e4m3").reshape(k, n)
        enc = None
    if enc is None:
        a_store = codes[:m * k].reshape(m, k)
        b_store = codes[m * k:].reshape(k, n)
    else:
        a_store, b_store = enc(av), enc(bv)
    a_store = a_store.T if transposed else a_store
    b_store = b_store.T if right_nk else b_store
    return (np.ascontiguousarray(a_store).reshape(-1), np.ascontiguousarray(b_store).reshape(-1),
            np.asarray(av, np.float64), np.asarray(bv, np.float64))


def _value(arr, dt):
    return O.bf16_to_f32(arr) if dt == dtypes.bfloat16 else arr.astype(np.float64)


@pytest.mark.parametrize("case", [
    dict(m=128, n=256, k=128, dtype=dtypes.bfloat16, kinds=["tgm_transpose16", "tgm_gemm_dense"]),
    dict(m=200, n=136, k=192, dtype=dtypes.float16, transposed=True, right_nk=True, activated=True,
         kinds=["tgm_transpose16", "tgm_gemm_dense", "kernel"]),
    dict(m=96, n=160, k=256, dtype=dtypes.fp8e4m3, right_nk=True, out_dtype=dtypes.float32, kinds=["tgm_gemm_fp8"]),
    dict(m=64, n=80, k=96, dtype=dtypes.float16, kinds=["kernel", "kernel", "tgm_gemm_dense"]),
    dict(m=48, n=72, k=200, dtype=dtypes.fp8e4m3, transposed=True, out_dtype=dtypes.float32,
         kinds=["kernel", "kernel", "tgm_gemm_fp8"]),
], ids=["bf16_row_major", "f16_kmajor_relu", "fp8_nk", "f16_k96_padded", "fp8_k200_padded"])
def test_scheduled_products_lowered_to_the_gemms(device, case):
    case = dict(case)
    kinds = case.pop("kinds")
    rng = np.random.default_rng(9)
    m, n, k, dt = case["m"], case["n"], case["k"], case["dtype"]
    a, b, av, bv = _operands(rng, m, n, k, dt, case.get("transposed", False), case.get("right_nk", False))
    sink = matrix_sink(**case)
    want = av @ bv
    if case.get("activated"):
        want = np.maximum(want, 0)
    out_dt = case.get("out_dtype") or dt
    lowered, linear = run_sink(device, sink, {1: a, 2: b}, lower=True)
    assert [c.src[0].arg.name if c.src[0].op is Ops.PROGRAM else "kernel" for c in linear.src] == kinds
    rendered, _ = run_sink(device, sink, {1: a, 2: b})
    for got in (lowered[0], rendered[0]):
        err = O.max_rel_err(_value(got, out_dt).reshape(m, n), want)
        assert err <= (1e-3 if out_dt == dtypes.float32 else 1e-2), err


def test_rebindable_inputs_are_staged(device):
    m, n, k = 64, 128, 64
    rng = np.random.default_rng(10)
    a, b, av, bv = _operands(rng, m, n, k, dtypes.float16, False, True)
    out, linear = run_sink(device, matrix_sink(m, n, k, dtypes.float16, right_nk=True), {1: a, 2: b}, lower=True,
                           input_slots=(1, 2))
    assert [c.src[0].op for c in linear.src] == [Ops.SINK, Ops.SINK, Ops.PROGRAM]
    assert O.max_rel_err(out[0].astype(np.float64).reshape(m, n), av @ bv) <= 1e-2


def test_compiled_kernels_are_cached_per_device(device):
    sink = elementwise(dtypes.float32, lambda x, y: x + y, 64, name="cached")
    assert compile_kernel(device, sink) is compile_kernel(device, sink)


def test_schedule_graph_replays_match_eager_runs(device):
    """A lowered schedule (transpose, GEMM, epilogue kernel) captured into one HIP graph: every
    replay, with new operands written between replays, equals the eager run of the same schedule."""
    m, n, k = 128, 192, 128
    sink = matrix_sink(m, n, k, dtypes.bfloat16, activated=True)
    params = sorted((u for u in sink.toposort() if u.op is Ops.PARAM), key=lambda u: u.arg.slot)
    bufs = [UOp.new_buffer(DEV, p.max_numel(), p.dtype) for p in params]
    linear = lower_matmul(UOp.linear(UOp.call(sink, *bufs)))
    bound = {b: device.allocator.alloc(p.max_numel() * 2) for p, b in zip(params, bufs)}
    graph = LinearGraph(device, linear, bound)
    assert len(graph.launches) == 3
    rng = np.random.default_rng(11)
    try:
        for _ in range(3):
            a, b, av, bv = _operands(rng, m, n, k, dtypes.bfloat16, False, False)
            device.allocator._copyin(bound[bufs[1]], memoryview(a).cast("B"))
            device.allocator._copyin(bound[bufs[2]], memoryview(b).cast("B"))
            graph(wait=True)
            replayed = np.empty(m * n, np.uint16)
            device.allocator._copyout(memoryview(replayed).cast("B"), bound[bufs[0]])
            run_linear(device, linear, graph.buffers, wait=True)
            eager = np.empty(m * n, np.uint16)
            device.allocator._copyout(memoryview(eager).cast("B"), bound[bufs[0]])
            np.testing.assert_array_equal(replayed, eager)
            want = np.maximum(av @ bv, 0)
            assert O.max_rel_err(O.bf16_to_f32(replayed).reshape(m, n), want) <= 1e-2
    finally:
        graph.close()


def test_long_reductions_fold_in_a_workgroup(device):
    """Row sums and maxima over 4096 points (one workgroup per row, LDS tree) and an RMSNorm
    whose every output point folds its row."""
    rows, cols = 97, 4096
    f32 = dtypes.float32
    x, o = UOp.param(1, f32, rows * cols, DEV), UOp.param(0, f32, rows, DEV)
    r, c = UOp.range(rows, 0), UOp.range(cols, 1, AxisType.REDUCE)
    v = x.index(r * cols + c)
    sink = o.index(r).store(v.reduce(c, arg=Ops.ADD) + v.reduce(c, arg=Ops.MAX) * 0.5).end(r).sink(
        arg=KernelInfo(name="rowfold"))
    assert "BARRIER" in [u.op.name for u in compile_kernel(device, sink).listing.uops]
    rng = np.random.default_rng(12)
    xs = rng.integers(-100, 100, rows * cols).astype(np.float32)  # integer-valued: the sums are exact
    out, _ = run_sink(device, sink, {1: xs})
    xm = xs.reshape(rows, cols)
    np.testing.assert_array_equal(out[0], xm.sum(1) + xm.max(1) * np.float32(0.5))
    # RMSNorm: y[r, k] = x[r, k] / sqrt(sum_j x[r, j]^2 / n + eps)
    n_rows, n = 8, 1000
    xx, yy = UOp.param(1, f32, n_rows * n, DEV), UOp.param(0, f32, n_rows * n, DEV)
    rr, kk, jj = UOp.range(n_rows, 0), UOp.range(n, 1), UOp.range(n, 2, AxisType.REDUCE)
    sq = xx.index(rr * n + jj)
    ms = (sq * sq).reduce(jj, arg=Ops.ADD) * (1.0 / n) + 1e-5
    norm = yy.index(rr * n + kk).store(xx.index(rr * n + kk) * ms.sqrt().reciprocal()).end(rr, kk).sink(
        arg=KernelInfo(name="rmsnorm"))
    xr = rng.standard_normal(n_rows * n).astype(np.float32)
    got, _ = run_sink(device, norm, {1: xr})
    want = xr.reshape(n_rows, n) / np.sqrt((xr.reshape(n_rows, n).astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-5)
    assert np.abs(got[0].reshape(n_rows, n) - want).max() <= 1e-5 * np.abs(want).max()


def _fp8_probe_values(target):
    """Every FP8 value, the midpoints between neighbours and the floats next to them, overflow
    thresholds, a wide random sweep, infinities, NaN and both zeros -- with both signs."""
    vals = O.fp8_decode(np.arange(256, dtype=np.uint8), target).astype(np.float64)
    fin = np.unique(vals[np.isfinite(vals) & (vals >= 0)])
    mids = (fin[1:] + fin[:-1]) / 2
    top = fin[-1] + (fin[-1] - fin[-2]) / 2  # halfway past the largest value
    pts = np.concatenate([fin, mids, [top, top * 1.01, 1e9]]).astype(np.float32)
    near = np.concatenate([np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(0))])
    rng = np.random.default_rng(13)
    sweep = (rng.standard_normal(4000) * np.exp2(rng.integers(-24, 20, 4000))).astype(np.float32)
    pos = np.concatenate([pts, near, np.abs(sweep), np.float32([np.inf, np.nan, 0.0])]).astype(np.float32)
    return np.concatenate([pos, -pos]).astype(np.float32)


@pytest.mark.parametrize("dt,target,torch_name", [(dtypes.fp8e4m3, "fp8e4m3", "float8_e4m3fn"),
                                                  (dtypes.fp8e5m2, "fp8e5m2", "float8_e5m2")], ids=["e4m3", "e5m2"])
def test_fp8_casts_stores_and_arithmetic_round_like_torch(device, dt, target, torch_name):
    """fp32 -> FP8 stores are bit-exact against torch's conversion on the CPU, and FP8 arithmetic
    is fp32 arithmetic rounded to the format after every operation."""
    import torch

    x = _fp8_probe_values(target)
    n = x.size
    i = UOp.range(n, 0)
    src, dst = UOp.param(1, dtypes.float32, n, DEV), UOp.param(0, dt, n, DEV)
    sink = dst.index(i).store(src.index(i).cast(dt)).end(i).sink(arg=KernelInfo(name=f"enc_{target}"))
    out, _ = run_sink(device, sink, {1: x})
    want = torch.from_numpy(x).to(getattr(torch, torch_name)).view(torch.uint8).numpy()
    bad = np.nonzero(out[0] != want)[0]
    assert bad.size == 0, (x[bad[:8]], out[0][bad[:8]], want[bad[:8]])
    # a * b + a with every operation rounded to the format
    rng = np.random.default_rng(14)
    codes = rng.integers(0, 256, (2, 2048)).astype(np.uint8)
    codes[(codes & 0x7F) >= (0x7C if target == "fp8e5m2" else 0x7F)] = 0x38  # finite operands
    sink2 = elementwise(dt, lambda a, b: a * b + a, 2048, name=f"arith_{target}")
    got, _ = run_sink(device, sink2, {1: codes[0], 2: codes[1]})
    f8 = getattr(torch, torch_name)
    a = torch.from_numpy(O.fp8_decode(codes[0], target))
    b = torch.from_numpy(O.fp8_decode(codes[1], target))
    ref = ((a * b).to(f8).float() + a).to(f8).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got[0], ref)
