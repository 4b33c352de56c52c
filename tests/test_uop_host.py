"""UOp kernels on the CPU: scheduled-matmul recognition and rewriting, the linearizer (run by a
CPU interpreter of its listings) and the HIP renderer (sources compiled for gfx950 here).

The matcher cases follow the reference's own (alexandreteles/tinygrad-dx12
test/backend/test_matmul_lowering.py:12-54: a 16 x 48 x 32 product, its transposed, activated
and float32 forms, a broadcast and a second output, explicit options).
"""

import shutil

import numpy as np
import pytest

import uop_interp
from tinygrad_mi355x.codegen.uop_matmul import lower_matmul, match_matmul
from tinygrad_mi355x.renderer.cstyle import MI355XRenderer
from tinygrad_mi355x.uop.linearize import linearize
from tinygrad_mi355x.uop.ops import AxisType, KernelInfo, Ops, UOp, dtypes

DEV = "MI355X"


def matrix_sink(m=16, n=48, k=32, dtype=dtypes.float16, transposed=False, activated=False, right_nk=False,
                out_dtype=None):
    """C[m, n] = sum_k A . B as a scheduled kernel (A [m, k] or, transposed, [k, m]; B [k, n] or,
    right_nk, [n, k]), products cast to fp32, the sum cast to the output dtype."""
    out_dtype = out_dtype or dtype
    output = UOp.param(0, out_dtype, m * n, DEV)
    left, right = UOp.param(1, dtype, m * k, DEV), UOp.param(2, dtype, k * n, DEV)
    row, col, inner = UOp.range(m, 1), UOp.range(n, 2), UOp.range(k, 0, AxisType.REDUCE)
    a = left.index(inner * m + row if transposed else row * k + inner)
    b = right.index(col * k + inner if right_nk else inner * n + col)
    if dtype.name.startswith("float8"):
        product = a.cast(dtypes.float32) * b.cast(dtypes.float32)
    else:
        product = (a * b).cast(dtypes.float32)
    value = product.reduce(inner, arg=Ops.ADD)
    if activated:
        value = value.maximum(0.0)
    value = value.cast(out_dtype)
    return output.index(row * n + col).store(value).end(row, col).sink(arg=KernelInfo(name="test"))


# ----------------------------------------------------------------------------- matcher
def test_recognizes_exact_row_major_matrix():
    spec = match_matmul(matrix_sink())
    assert spec is not None
    assert (spec.m, spec.n, spec.k) == (16, 48, 32)
    assert tuple(p.arg.slot for p in (spec.output, spec.left, spec.right)) == (0, 1, 2)
    assert spec.transposed == (False, False) and not spec.epilogue


@pytest.mark.parametrize("kwargs", [{"transposed": True}, {"activated": True}, {"dtype": dtypes.float32},
                                    {"right_nk": True}])
def test_recognizes_native_matrix_semantics(kwargs):
    spec = match_matmul(matrix_sink(**kwargs))
    assert spec is not None
    assert spec.transposed == (kwargs.get("transposed", False), kwargs.get("right_nk", False))
    assert spec.epilogue == kwargs.get("activated", False)
    assert spec.left.dtype == kwargs.get("dtype", dtypes.float16)


def test_rejects_broadcast_and_second_output():
    ast = matrix_sink()
    row = ast.src[0].src[1]
    assert match_matmul(ast.substitute({row: row.const_like(0)})) is None
    assert match_matmul(ast.replace(src=ast.src * 2)) is None


def test_rejects_explicit_codegen_options_and_aliasing():
    assert match_matmul(matrix_sink().replace(arg=KernelInfo(opts_to_apply=()))) is None
    ast = matrix_sink()
    out_param = ast.src[0].src[0].src[0].src[0]
    left = next(u for u in ast.toposort() if u.op is Ops.PARAM and u.arg.slot == 1)
    assert match_matmul(ast.substitute({left: out_param})) is None  # output aliases an input
    small = UOp.param(1, dtypes.float16, 16 * 32 - 1, DEV)
    assert match_matmul(ast.substitute({left: small})) is None     # too small for m x k


def test_rejects_non_affine_and_product_of_axes():
    ast = matrix_sink()
    store = ast.src[0].src[0]
    row, col = ast.src[0].src[1:]
    bad = store.src[0].src[0].index(row * col)
    assert match_matmul(ast.substitute({store.src[0]: bad})) is None


# ----------------------------------------------------------------------------- rewrite
def _buffers(*specs):
    return [UOp.new_buffer(DEV, n, dt) for n, dt in specs]


def _kinds(linear):
    return [c.src[0].arg.name if c.src[0].op is Ops.PROGRAM else "kernel" for c in linear.src]


def test_lowering_plans_transposes_product_and_epilogue():
    m, n, k = 128, 256, 128
    out, a, b = _buffers((m * n, dtypes.bfloat16), (m * k, dtypes.bfloat16), (k * n, dtypes.bfloat16))
    plain = lower_matmul(UOp.linear(UOp.call(matrix_sink(m, n, k, dtypes.bfloat16), out, a, b)))
    assert _kinds(plain) == ["tgm_transpose16", "tgm_gemm_dense"]    # B [K, N] -> [N, K]
    assert plain.src[1].src[1] is out                                   # product straight into C
    nk = lower_matmul(UOp.linear(UOp.call(matrix_sink(m, n, k, dtypes.bfloat16, right_nk=True), out, a, b)))
    assert _kinds(nk) == ["tgm_gemm_dense"]
    both = lower_matmul(UOp.linear(UOp.call(matrix_sink(m, n, k, dtypes.bfloat16, transposed=True,
                                                        right_nk=True), out, a, b)))
    assert _kinds(both) == ["tgm_transpose16", "tgm_gemm_dense"]
    act = lower_matmul(UOp.linear(UOp.call(matrix_sink(m, n, k, dtypes.bfloat16, activated=True,
                                                       right_nk=True), out, a, b)))
    assert _kinds(act) == ["tgm_gemm_dense", "kernel"]
    tmp = act.src[0].src[1]
    assert tmp.dtype == dtypes.float32 and act.src[1].src[-1] is tmp    # epilogue reads the fp32 product
    epi = act.src[1].src[0]
    assert not any(u.op is Ops.REDUCE for u in epi.toposort())
    out32, a8, b8 = _buffers((m * n, dtypes.float32), (m * k, dtypes.fp8e4m3), (k * n, dtypes.fp8e4m3))
    fp8 = lower_matmul(UOp.linear(UOp.call(matrix_sink(m, n, k, dtypes.fp8e4m3, right_nk=True,
                                                       out_dtype=dtypes.float32), out32, a8, b8)))
    assert _kinds(fp8) == ["tgm_gemm_fp8"]


def test_plan_rejects_program_buffers_smaller_than_the_kernel_touches():
    """A hand-built LINEAR may bind a library PROGRAM's slots to BUFFERs whose own sizes are
    consistent but smaller than the product the program was built for; plan() must refuse it
    before anything is launched (the kernel would read and write past those buffers)."""
    from tinygrad_mi355x.codegen import program as P
    from tinygrad_mi355x.runtime import ops_mi355x as R
    from tinygrad_mi355x.runtime.schedule import plan

    class FakeDev:
        device = DEV

    dev = FakeDev()
    m, n, k = 128, 256, 128
    prog = P.dense_program("bfloat16", m, k, "bfloat16", n, k, k, "bfloat16", n)
    assert prog.slot_bytes == (m * n * 2, m * k * 2, n * k * 2)

    def bound(specs):
        uops = _buffers(*specs)
        return uops, {u: R.MI355XBuffer(dev, R._Allocation(0x1000 * (i + 1), nb * 2), nb * 2)
                      for i, (u, (nb, _)) in enumerate(zip(uops, specs))}

    full, bufs = bound([(m * n, dtypes.bfloat16), (m * k, dtypes.bfloat16), (n * k, dtypes.bfloat16)])
    launches, _ = plan(dev, UOp.linear(UOp.call(UOp(Ops.PROGRAM, None, (), prog), *full)), bufs)
    assert len(launches) == 1 and launches[0].native
    for short in range(3):
        specs = [(m * n, dtypes.bfloat16), (m * k, dtypes.bfloat16), (n * k, dtypes.bfloat16)]
        specs[short] = (specs[short][0] // 2, dtypes.bfloat16)
        small, bufs = bound(specs)
        with pytest.raises(ValueError, match="the kernel touches"):
            plan(dev, UOp.linear(UOp.call(UOp(Ops.PROGRAM, None, (), prog), *small)), bufs)


def test_lowering_pads_k_and_keeps_products_without_a_native_kernel():
    m, n, k = 64, 64, 96
    out, a, b = _buffers((m * n, dtypes.float16), (m * k, dtypes.float16), (k * n, dtypes.float16))
    call = UOp.call(matrix_sink(m, n, k), out, a, b)
    padded = lower_matmul(UOp.linear(call))                               # K % 64 != 0: zero columns to 128
    assert _kinds(padded) == ["kernel", "kernel", "tgm_gemm_dense"]
    assert [c.src[1].max_numel() for c in padded.src[:2]] == [m * 128, n * 128]
    # the padding kernel: [rows, k] or K-major [k, rows] -> [rows, kp], zero past column k
    rows, kk, kp = 3, 5, 8
    src = np.arange(rows * kk, dtype=np.int32) + 1
    for k_major in (False, True):
        _, buf = _pad_operand(rows, kk, kp, k_major)
        dst = np.full(rows * kp, -1, np.int32)
        uop_interp.run(linearize(buf), {0: dst, 1: src})
        stored = src.reshape(kk, rows).T if k_major else src.reshape(rows, kk)
        np.testing.assert_array_equal(dst.reshape(rows, kp), np.pad(stored, ((0, 0), (0, kp - kk))))
    buffers32 = _buffers((64 * 64, dtypes.float32), (64 * 64, dtypes.float32), (64 * 64, dtypes.float32))
    call32 = UOp.call(matrix_sink(64, 64, 64, dtypes.float32), *buffers32)
    assert _kinds(lower_matmul(UOp.linear(call32))) == ["kernel"]        # fp32 operands


def _pad_operand(rows, k, kp, k_major):
    from tinygrad_mi355x.codegen.uop_matmul import _pad_call

    call, staged = _pad_call(DEV, UOp.new_buffer(DEV, rows * k, dtypes.int32), dtypes.int32, rows, k, kp, k_major)
    return staged, call.src[0]


def test_lowering_stages_rebindable_inputs():
    m, n, k = 64, 128, 64
    out, a, b = _buffers((m * n, dtypes.float16), (m * k, dtypes.float16), (k * n, dtypes.float16))
    call = UOp.call(matrix_sink(m, n, k, right_nk=True), out, a, b)
    staged = lower_matmul(UOp.linear(call), input_uops=(a,))
    assert _kinds(staged) == ["kernel", "tgm_gemm_dense"]
    copy = staged.src[0]
    assert copy.src[2] is a and staged.src[1].src[2] is copy.src[1]
    # an output that is a rebindable input keeps its ordinary kernel
    assert _kinds(lower_matmul(UOp.linear(call), input_uops=(out,))) == ["kernel"]
    # so does a call whose arguments do not hold their parameters (too small, another dtype)
    small = _buffers((m * k - 1, dtypes.float16))[0]
    assert _kinds(lower_matmul(UOp.linear(UOp.call(matrix_sink(m, n, k, right_nk=True), out, small, b)))) == ["kernel"]
    wrong = _buffers((m * k, dtypes.bfloat16))[0]
    assert _kinds(lower_matmul(UOp.linear(UOp.call(matrix_sink(m, n, k, right_nk=True), out, wrong, b)))) == ["kernel"]
    # so does a call that binds one buffer as both the output and an operand
    square = _buffers((m * m, dtypes.float16))[0]
    inplace = UOp.call(matrix_sink(m, m, m, right_nk=True), square, square, b)
    assert _kinds(lower_matmul(UOp.linear(inplace))) == ["kernel"]


# ----------------------------------------------------------------------------- linearizer
def test_linearized_matmul_and_epilogue_run_on_the_interpreter():
    rng = np.random.default_rng(0)
    m, n, k = 5, 7, 9
    a = rng.integers(-4, 5, m * k).astype(np.float32)
    b = rng.integers(-4, 5, k * n).astype(np.float32)
    out = np.zeros(m * n, np.float32)
    uop_interp.run(linearize(matrix_sink(m, n, k, dtypes.float32, activated=True)), {0: out, 1: a, 2: b})
    want = np.maximum(a.reshape(m, k) @ b.reshape(k, n), 0)
    np.testing.assert_array_equal(out.reshape(m, n), want)


def test_linearized_nested_reductions_hoist_and_gates():
    """Row sums of a gated (padded) read, scaled by a value loaded once per row, then the max
    over a variable-length second reduction."""
    rows, cols, pad = 6, 10, 7
    x, s, o = UOp.param(1, dtypes.int32, rows * pad), UOp.param(2, dtypes.int32, rows), UOp.param(0, dtypes.int32, rows)
    r, c, j = UOp.range(rows, 0), UOp.range(cols, 1, AxisType.REDUCE), UOp.range(UOp.variable("n", 1, 8), 2,
                                                                                  AxisType.REDUCE)
    gated = x.index(r * pad + c, c < pad)
    total = (gated * s.index(r)).reduce(c, arg=Ops.ADD)
    peak = x.index(r * pad + (j % pad)).reduce(j, arg=Ops.MAX)
    sink = o.index(r).store(total + peak).end(r).sink(arg=KernelInfo(name="rows"))
    listing = linearize(sink)
    assert [v.arg[0] for v in listing.variables] == ["n"]
    xs = np.arange(rows * pad, dtype=np.int32) - 20
    sc = np.arange(rows, dtype=np.int32) + 1
    out = np.zeros(rows, np.int32)
    uop_interp.run(listing, {0: out, 1: xs, 2: sc}, {"n": 5})
    xm = xs.reshape(rows, pad)
    np.testing.assert_array_equal(out, xm.sum(1) * sc + xm[:, :5].max(1))
    # the scale is loop-invariant: read once per work-item, before the column loop
    ops = [u.op.name for u in listing.uops]
    first_range = ops.index("RANGE")
    scale_loads = [i for i, u in enumerate(listing.uops) if u.op is Ops.LOAD and u.src[0].src[0].op is Ops.PARAM and u.src[0].src[0].arg.slot == 2]
    assert len(scale_loads) == 1 and scale_loads[0] < first_range


def test_invariant_loads_stay_inside_loops_that_may_not_run():
    """A REDUCE over a variable bound n >= 0 whose body reads s[n - 1] (loop-invariant): at n = 0
    the loop runs no iteration and the kernel must not read s[-1]; with a constant bound > 0 the
    invariant load still moves ahead of the loop."""
    rows, width = 3, 4
    x, s, o = UOp.param(1, dtypes.int32, rows * width), UOp.param(2, dtypes.int32, width), UOp.param(0, dtypes.int32, rows)
    n = UOp.variable("n", 0, width)
    r, j = UOp.range(rows, 0), UOp.range(n, 1, AxisType.REDUCE)
    total = (x.index(r * width + j) * s.index(n - 1)).reduce(j, arg=Ops.ADD)
    listing = linearize(o.index(r).store(total).end(r).sink(arg=KernelInfo(name="tail")))
    xs, sc = np.arange(rows * width, dtype=np.int32) + 1, np.array([2, 3, 5, 7], np.int32)
    for nv in range(width + 1):
        out = np.full(rows, -1, np.int32)
        uop_interp.run(listing, {0: out, 1: xs, 2: sc}, {"n": nv})
        want = xs.reshape(rows, width)[:, :nv].sum(1) * (sc[nv - 1] if nv else 0)
        np.testing.assert_array_equal(out, want)
    loads = [i for i, u in enumerate(listing.uops) if u.op is Ops.LOAD and u.src[0].src[0].op is Ops.PARAM
             and u.src[0].src[0].arg.slot == 2]
    inner = [i for i, u in enumerate(listing.uops) if u.op is Ops.RANGE][-1]
    assert loads and all(i > inner for i in loads)
    fixed = (x.index(r * width + UOp.range(width, 1, AxisType.REDUCE)) * s.index(r)).reduce(
        UOp.range(width, 1, AxisType.REDUCE), arg=Ops.ADD)
    hoisted = linearize(o.index(r).store(fixed).end(r).sink(arg=KernelInfo(name="fixed")))
    loads = [i for i, u in enumerate(hoisted.uops) if u.op is Ops.LOAD and u.src[0].src[0].op is Ops.PARAM
             and u.src[0].src[0].arg.slot == 2]
    inner = [i for i, u in enumerate(hoisted.uops) if u.op is Ops.RANGE][-1]
    assert len(loads) == 1 and loads[0] < inner


def test_linearizer_rejects_malformed_kernels():
    o, r = UOp.param(0, dtypes.float32, 4), UOp.range(4, 0)
    stray = UOp.range(4, 1)
    with pytest.raises(ValueError):
        linearize(o.index(r).store(stray.cast(dtypes.float32)).end(r).sink())      # range outside its loop
    with pytest.raises(ValueError):
        linearize(o.index(r).store(1.0).end(UOp.range(4, 2, AxisType.REDUCE)).sink())
    with pytest.raises(ValueError):
        linearize(UOp.param(0, dtypes.float32, 2**31).index(r).store(1.0).end(r).sink())


# ----------------------------------------------------------------------------- renderer
needs_compiler = pytest.mark.skipif(shutil.which("hipcc") is None and not __import__("os").path.exists(
    "/opt/rocm/bin/amdclang++"), reason="no ROCm compiler")


def _elementwise(dt, fn, n=64, out_dt=None):
    a, b = UOp.param(1, dt, n), UOp.param(2, dt, n)
    o = UOp.param(0, out_dt or dt, n)
    i = UOp.range(n, 0)
    return o.index(i).store(fn(a.index(i), b.index(i))).end(i).sink(arg=KernelInfo(name=f"ew_{dt.name}"))


@needs_compiler
def test_rendered_kernels_compile_for_gfx950():
    r = MI355XRenderer()
    sinks = [_elementwise(dt, lambda x, y: (x * y + x).maximum(y) - (x < y).where(x, y))
             for dt in (dtypes.int8, dtypes.uint16, dtypes.int32, dtypes.uint64, dtypes.float16, dtypes.bfloat16,
                        dtypes.float32, dtypes.float64)]
    sinks.append(_elementwise(dtypes.float32, lambda x, y: (x.exp2() + y.log2() + x.sqrt() + y.sin()).reciprocal()))
    sinks.append(_elementwise(dtypes.int32, lambda x, y: (x << 3) ^ (y >> 1) | (x & y) // 7 % 5))
    sinks.append(_elementwise(dtypes.fp8e4m3, lambda x, y: x.cast(dtypes.float32) + y.cast(dtypes.float32),
                              out_dt=dtypes.float32))
    sinks.append(_elementwise(dtypes.bool, lambda x, y: x.ne(y), out_dt=dtypes.bool))
    sinks.append(_elementwise(dtypes.float32, lambda x, y: x.bitcast(dtypes.int32).cast(dtypes.float32) + y,
                              out_dt=dtypes.float32))
    sinks.append(matrix_sink(16, 48, 32, activated=True))
    for sink in sinks:
        src = r.render(linearize(sink))
        obj = r.compiler.compile(src)
        assert len(obj) > 1000 and 'extern "C" __global__' in src


def test_renderer_literals_and_dtype_rules():
    r = MI355XRenderer()
    src = r.render(linearize(_elementwise(dtypes.bfloat16, lambda x, y: x * y + UOp.const(dtypes.bfloat16, -0.0))))
    assert "(float)" in src and "-0x0.0p+0f" in src         # bf16: fp32 arithmetic, -0.0 kept
    src = r.render(linearize(_elementwise(dtypes.int32, lambda x, y: x + y)))
    assert "(unsigned int)" in src                           # signed add wraps (no overflow UB)
    src = r.render(linearize(_elementwise(dtypes.bool, lambda x, y: x.ne(y), out_dt=dtypes.bool)))
    assert "!= 0" in src and "? 1 : 0" in src               # bool storage is a byte
    inf = UOp.const(dtypes.float32, float("inf"))
    src = r.render(linearize(_elementwise(dtypes.float32, lambda x, y: x.maximum(inf))))
    assert "__builtin_inff()" in src and "fmaxf" in src
    assert "const float* __restrict__ data1" in src and "float* __restrict__ data0" in src


def test_renderer_takes_tinygrad_spelled_listings():
    """A listing spelled with tinygrad's names (DEFINE_GLOBAL with an integer slot, pointer dtypes
    with a ``base``, dtype names "float" / "int") renders like its own."""
    from types import SimpleNamespace as NS

    def op(name):
        return NS(name=name)

    f32, i32 = NS(name="float"), NS(name="int")
    ptr = NS(base=f32)
    g0 = NS(op=op("DEFINE_GLOBAL"), dtype=ptr, src=(), arg=0)
    g1 = NS(op=op("DEFINE_GLOBAL"), dtype=ptr, src=(), arg=1)
    n64 = NS(op=op("CONST"), dtype=i32, src=(), arg=64)
    lid = NS(op=op("SPECIAL"), dtype=i32, src=(n64,), arg="lidx0")
    ld_idx = NS(op=op("INDEX"), dtype=ptr, src=(g1, lid), arg=None)
    ld = NS(op=op("LOAD"), dtype=f32, src=(ld_idx,), arg=None)
    two = NS(op=op("CONST"), dtype=f32, src=(), arg=2.0)
    mul = NS(op=op("MUL"), dtype=f32, src=(ld, two), arg=None)
    st_idx = NS(op=op("INDEX"), dtype=ptr, src=(g0, lid), arg=None)
    st = NS(op=op("STORE"), dtype=None, src=(st_idx, mul), arg=None)
    src = MI355XRenderer().render([g0, g1, n64, lid, ld_idx, ld, two, mul, st_idx, st])
    assert "__launch_bounds__(64)" in src and "float* __restrict__ data0" in src and "0x1.0000000000000p+1f" in src


def test_long_reductions_fold_in_a_workgroup():
    """Reductions of at least 256 points: one workgroup per stored point, work-items striding over
    the points (the last chunk's surplus folds the identity), then an LDS halving tree."""
    rows, cols, a, b = 3, 1000, 20, 30
    x = UOp.param(1, dtypes.int32, rows * cols)
    y = UOp.param(2, dtypes.int32, rows * a * b)
    o = UOp.param(0, dtypes.int32, rows)
    r = UOp.range(rows, 0)
    c = UOp.range(cols, 1, AxisType.REDUCE)
    i, j = UOp.range(a, 2, AxisType.REDUCE), UOp.range(b, 3, AxisType.REDUCE)
    total = x.index(r * cols + c).reduce(c, arg=Ops.ADD)
    peak = (y.index(r * (a * b) + i * b + j) * (i + 1)).reduce(i, j, arg=Ops.MAX)
    sink = o.index(r).store(total * 3 + peak).end(r).sink(arg=KernelInfo(name="long"))
    listing = linearize(sink)
    assert listing.global_size == (rows, 1, 1) and listing.local_size == (256, 1, 1)
    names = [u.op.name for u in listing.uops]
    assert names.count("DEFINE_LOCAL") == 2 and names.count("BARRIER") == 2 * 9
    rng = np.random.default_rng(3)
    xs = rng.integers(-1000, 1000, rows * cols).astype(np.int32)
    ys = rng.integers(-1000, 1000, rows * a * b).astype(np.int32)
    out = np.zeros(rows, np.int32)
    uop_interp.run(listing, {0: out, 1: xs, 2: ys})
    weights = np.arange(1, a + 1, dtype=np.int32)[:, None]
    want = xs.reshape(rows, cols).sum(1) * 3 + (ys.reshape(rows, a, b) * weights).reshape(rows, -1).max(1)
    np.testing.assert_array_equal(out, want)
    # short reductions keep one work-item per stored point
    short = o.index(r).store(x.index(r * cols + UOp.range(100, 4, AxisType.REDUCE)).reduce(
        UOp.range(100, 4, AxisType.REDUCE), arg=Ops.ADD)).end(r).sink(arg=KernelInfo(name="short"))
    assert "BARRIER" not in [u.op.name for u in linearize(short).uops]


def test_one_renderer_renders_uop_listings_from_many_threads():
    """Listings rendered from several threads at once equal their single-threaded renders."""
    import threading

    r = MI355XRenderer()
    kinds = (dtypes.float32, dtypes.float64, dtypes.int32, dtypes.float16, dtypes.bfloat16, dtypes.uint8)
    listings = []
    for i in range(12):
        dt = kinds[i % len(kinds)]
        src, out = UOp.param(1, dt, 4 + i), UOp.param(0, dt, 4 + i)
        k = UOp.range(4 + i, 0)
        v = src.index(k)
        for _ in range(200 * (1 + i % 4)):
            v = v * src.index(k) + src.index(k)
        listings.append(linearize(out.index(k).store(v).end(k).sink(arg=KernelInfo(name=f"chain_{i}"))))
    alone = [r.render(x) for x in listings]
    start = threading.Event()
    results: dict[int, list] = {}

    def worker(i: int) -> None:
        start.wait()
        results[i] = [r.render(listings[i]) for _ in range(3)]

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(listings))]
    for t in threads:
        t.start()
    start.set()
    for t in threads:
        t.join(60)
    assert all(results[i] == [alone[i]] * 3 for i in range(len(listings)))


def test_in_place_updates_and_deep_expression_chains():
    """One INDEX both read and written through (x[i] = x[i] * 3 + 1), and a 5000-deep chain of
    operations (listed without recursion)."""
    n = 10
    x = UOp.param(0, dtypes.int32, n)
    i = UOp.range(n, 0)
    buf = np.arange(n, dtype=np.int32)
    uop_interp.run(linearize(x.index(i).store(x.index(i) * 3 + 1).end(i).sink()), {0: buf})
    np.testing.assert_array_equal(buf, np.arange(n) * 3 + 1)
    y, o = UOp.param(1, dtypes.int32, n), UOp.param(0, dtypes.int32, n)
    v = y.index(i)
    for _ in range(5000):
        v = v + 1
    out = np.zeros(n, np.int32)
    listing = linearize(o.index(i).store(v).end(i).sink())
    uop_interp.run(listing, {0: out, 1: np.arange(n, dtype=np.int32)})
    np.testing.assert_array_equal(out, np.arange(n) + 5000)
    assert "data0" in MI355XRenderer().render(listing)


def test_graphs_built_in_many_threads_share_their_nodes():
    """Hash-consing holds across threads: the same expression built concurrently is one object."""
    import threading

    results = []
    start = threading.Event()

    def build() -> None:
        start.wait()
        x = UOp.param(3, dtypes.float32, 64)
        i = UOp.range(64, 7)
        v = x.index(i)
        for _ in range(300):
            v = v * 2.0 + x.index(i)
        results.append(v)

    threads = [threading.Thread(target=build) for _ in range(8)]
    for t in threads:
        t.start()
    start.set()
    for t in threads:
        t.join(60)
    assert len(results) == 8 and all(r is results[0] for r in results)
