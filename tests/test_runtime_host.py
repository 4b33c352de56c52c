"""Host-side checks of the device plugin: compiler, renderer, signatures and argument
validation (no GPU needed; mirrors the spirit of the reference's test_toolchain.py and
the argument checks of ops_dx12.py:659-744)."""

import struct

import pytest
import torch

from tinygrad_mi355x.renderer.cstyle import BufferParam, KernelSpec, MI355XRenderer
from tinygrad_mi355x.runtime import ops_mi355x as R
from tinygrad_mi355x.runtime.support.compiler_hip import (CompileError, KernelSignature, MI355XCompiler,
                                                          parse_signature, unpack_object)

VADD = KernelSpec("vadd", (BufferParam("out", torch.float32, True), BufferParam("a", torch.float32),
                           BufferParam("b", torch.float32)), (("n", "i32"),),
                  ("const int i = gidx0 * 256 + lidx0;", "if (i < n) out[i] = a[i] + b[i];"))


def test_renderer_output_compiles_to_a_gfx950_code_object():
    r = MI355XRenderer()
    src = r.render(VADD)
    obj = r.compiler.compile(src)
    source, sig, code = unpack_object(obj)
    assert source == src
    assert sig == KernelSignature("vadd", ("ptr", "ptr", "ptr", "i32"))
    assert code[:4] == b"\x7fELF"
    assert r.compiler.compile(src) is obj  # cached by source


def test_compiler_cache_key_is_deterministic_and_settings_dependent():
    assert MI355XCompiler().cachekey == MI355XCompiler().cachekey
    assert MI355XCompiler().cachekey != MI355XCompiler(opt="-O2").cachekey
    assert MI355XCompiler().cachekey.startswith("mi355x_")


def test_compile_error_carries_diagnostics():
    bad = '#include <hip/hip_runtime.h>\nextern "C" __global__ void k(float* o) { o[0] = undefined_name; }\n'
    with pytest.raises(CompileError, match="undefined_name"):
        MI355XCompiler().compile(bad)


def test_signature_parsing():
    src = ('extern "C" __global__ void __launch_bounds__(128) f(const unsigned char* __restrict__ w, float* y, '
           'long long n, unsigned int k, float alpha, double beta) {}')
    sig = parse_signature(src)
    assert sig.params == ("ptr", "ptr", "i64", "u32", "f32", "f64")
    assert (sig.buffers, sig.scalars) == (2, 4)
    with pytest.raises(CompileError):
        parse_signature('extern "C" __global__ void g(struct S s) {}')
    with pytest.raises(CompileError):
        parse_signature("__global__ void not_extern_c(float* x) {}")


def test_renderer_rejects_bad_specs():
    r = MI355XRenderer()
    with pytest.raises(ValueError):
        r.render(KernelSpec("k", (BufferParam("x", torch.complex64),)))
    with pytest.raises(ValueError):
        r.render(KernelSpec("k", (BufferParam("x", torch.float32),), local_size=(2048, 1, 1)))
    with pytest.raises(ValueError):
        r.render(KernelSpec("k", (BufferParam("x", torch.float32),), (("n", "i8"),)))
    assert torch.bfloat16 in r.supported_dtypes() and r.shared_max == 160 * 1024


class _FakeDev:
    """Stands in for a device in checks that must fail before any HIP call."""

    device = "MI355X"


def _fake_program(params):
    prog = object.__new__(R.MI355XProgram)
    prog.dev, prog.name = _FakeDev(), "k"
    prog.signature = KernelSignature("k", tuple(params))
    return prog


def _fake_buffer(dev, size=64):
    return R.MI355XBuffer(dev, R._Allocation(0x1000, size), size)


def test_program_argument_validation_happens_before_launch():
    prog = _fake_program(("ptr", "ptr", "i32"))
    a, b = _fake_buffer(prog.dev), _fake_buffer(prog.dev)
    with pytest.raises(ValueError, match="dispatch dimensions"):
        prog(a, b, global_size=(1, 1), vals=(1,))
    with pytest.raises(ValueError, match="dispatch dimensions"):
        prog(a, b, global_size=(1, 70000, 1), vals=(1,))
    with pytest.raises(ValueError, match="workgroup"):
        prog(a, b, local_size=(1025, 1, 1), vals=(1,))
    with pytest.raises(ValueError, match="signature mismatch"):
        prog(a, vals=(1,))
    with pytest.raises(ValueError, match="signature mismatch"):
        prog(a, _fake_buffer(_FakeDev()), vals=(1,))  # buffer of another device
    with pytest.raises(ValueError, match="scalar argument count"):
        prog(a, b, vals=())
    # zero work is skipped entirely (no HIP call): None, or 0.0 seconds when waiting
    assert prog(a, b, global_size=(0, 1, 1), vals=()) is None
    assert prog(a, b, global_size=(4, 0, 1), vals=(), wait=True) == 0.0


def test_kernarg_layout_follows_natural_alignment():
    prog = _fake_program(("ptr", "i32", "ptr", "f32", "f64"))
    a = R.MI355XBuffer(prog.dev, R._Allocation(0x1000, 64), 64, 16)
    b = R.MI355XBuffer(prog.dev, R._Allocation(0x2000, 64), 64)
    args = prog._kernargs((a, b), (7, 1.5, 2.25))
    assert len(args) == 40
    assert struct.unpack_from("<Q", args, 0)[0] == 0x1010
    assert struct.unpack_from("<i", args, 8)[0] == 7
    assert struct.unpack_from("<Q", args, 16)[0] == 0x2000
    assert struct.unpack_from("<f", args, 24)[0] == 1.5
    assert struct.unpack_from("<d", args, 32)[0] == 2.25


def test_allocator_checks_need_no_gpu():
    alloc = object.__new__(R.MI355XAllocator)
    dev = _FakeDev()
    alloc.dev = dev
    buf = _fake_buffer(dev, 64)
    view = alloc._offset(buf, 16, 8)
    assert (view.size, view.offset, view.owner) == (16, 8, buf.owner)
    nested = alloc._offset(view, 8, 8)
    assert nested.address == 0x1000 + 16
    for size, offset in ((65, 0), (8, 60), (-1, 0), (4, -1)):
        with pytest.raises(ValueError, match="outside allocation"):
            alloc._offset(buf, size, offset)
    with pytest.raises(ValueError, match="external_ptr"):
        alloc._alloc(16, R.BufferSpec(external_ptr=0x1234))
    with pytest.raises(ValueError, match="upload exceeds"):
        alloc._copyin(view, memoryview(bytes(17)))
    with pytest.raises(ValueError, match="readback exceeds"):
        alloc._copyout(memoryview(bytearray(17)), view)
    with pytest.raises(ValueError, match="transfer exceeds"):
        alloc._transfer(view, buf, 32, dev, dev)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU failure")
def test_opening_a_device_without_a_gpu_raises():
    with pytest.raises(RuntimeError):
        R.MI355XDevice("MI355X")


def test_graph_validation_without_a_gpu():
    """MI355XGraph rejects empty sequences and programs of several devices before touching HIP."""
    from types import SimpleNamespace

    from tinygrad_mi355x.runtime.graph import MI355XGraph, StreamGraph

    with pytest.raises(ValueError, match="at least one"):
        MI355XGraph([])
    a, b = SimpleNamespace(dev=object()), SimpleNamespace(dev=object())
    with pytest.raises(ValueError, match="one device"):
        MI355XGraph([(a, (), (1, 1, 1), (1, 1, 1), ()), (b, (), (1, 1, 1), (1, 1, 1), ())])
    with pytest.raises(ValueError, match="non-null"):
        StreamGraph(lambda: None, 0)


def test_shared_renderer_concurrent_sources():
    """Concurrent callers of one renderer receive exactly their sequential source (the reference's
    test_renderer_concurrency.py:11-36 idea): 8 kernels of 4 dtypes with long bodies, rendered
    from 8 threads released together."""
    from concurrent.futures import ThreadPoolExecutor
    from threading import Barrier

    r = MI355XRenderer()
    cases = []
    for slot in range(8):
        dt = (torch.float32, torch.float64, torch.int32, torch.float16)[slot % 4]
        body = ["auto v = src[0];"] + ["v = v * v + src[0];"] * 2048 + ["out[0] = v;"]
        cases.append(KernelSpec(f"thread_{slot}", (BufferParam("out", dt, True), BufferParam("src", dt)), (),
                                tuple(body)))
    expected = [r.render(c) for c in cases]
    barrier = Barrier(len(cases))

    def render(slot: int) -> str:
        barrier.wait()
        try:
            return r.render(cases[slot])
        except Exception as error:  # noqa: BLE001 - a failure must show up as a mismatch
            return type(error).__name__

    with ThreadPoolExecutor(max_workers=len(cases)) as workers:
        actual = list(workers.map(render, range(len(cases))))
    assert actual == expected

