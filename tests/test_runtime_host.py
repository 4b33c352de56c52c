"""Host-side checks of the device plugin: compiler, renderer, signatures and argument
validation (no GPU needed; mirrors the spirit of the reference's test_toolchain.py and
the argument checks of ops_dx12.py:659-744)."""

import struct
import subprocess
from pathlib import Path

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
    assert {"bfloat16", "float8_e4m3fn", "float8_e5m2"} <= r.supported_dtypes() and r.shared_max == 160 * 1024


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


def test_one_renderer_serves_many_threads():
    """Threads that share one renderer each get the source they would get alone.  Twelve kernel
    specifications differ in name, parameter count, dtypes and body length (up to a few thousand
    statements, so renders overlap in time); each thread renders its own spec three times after
    a common start signal, and every result must equal the single-threaded render."""
    import threading

    r = MI355XRenderer()
    kinds = (torch.float16, torch.int64, torch.bfloat16, torch.float32, torch.uint8, torch.float64)
    specs = []
    for i in range(12):
        dt = kinds[i % len(kinds)]
        params = (BufferParam("dst", dt, True),) + tuple(BufferParam(f"in{j}", dt) for j in range(1 + i % 3))
        body = ("auto acc = in0[gidx0];",) + ("acc = acc + in0[gidx0];",) * (300 * (i + 1)) + ("dst[gidx0] = acc;",)
        specs.append(KernelSpec(f"accumulate_{i}", params, (("n", "i64"),) if i % 2 else (), body))
    alone = [r.render(spec) for spec in specs]
    start = threading.Event()
    results: dict[int, list] = {}

    def worker(i: int) -> None:
        start.wait()
        out = []
        for _ in range(3):
            try:
                out.append(r.render(specs[i]))
            except Exception as error:  # noqa: BLE001 -- recorded so that a failure reads as a mismatch
                out.append(repr(error))
        results[i] = out

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(specs))]
    for t in threads:
        t.start()
    start.set()
    for t in threads:
        t.join(60)
    assert sorted(results) == list(range(len(specs)))
    for i, got in results.items():
        assert got == [alone[i]] * 3, specs[i].name


class _StubHip:
    """A HIP binding with no GPU behind it: every call succeeds, except the names the test
    arms to fail once; host allocations are real host memory so staging copies can run."""

    H2D, D2H, D2D = 1, 2, 3

    def __init__(self) -> None:
        self.calls: list[str] = []
        self.armed: set[str] = set()
        self._events = 0
        self._host: dict[int, object] = {}

    def call(self, name: str, *args) -> None:
        self.calls.append(name)
        if name in self.armed:
            self.armed.discard(name)
            raise RuntimeError(f"{name} failed: 1 (injected)")
        if name == "hipHostFree":
            self._host.pop(args[0], None)

    def launch(self, function, grid, block, kernargs, stream, shared=0) -> None:
        self.call("hipModuleLaunchKernel", function, *grid, *block, shared, stream)

    def event_create(self) -> int:
        self._events += 1
        return self._events

    def host_malloc(self, size: int) -> int:
        import ctypes

        buf = ctypes.create_string_buffer(max(size, 1))
        self._host[ctypes.addressof(buf)] = buf
        return ctypes.addressof(buf)

    def query(self, name: str, handle: int) -> bool:
        return True

    def set_device(self, ordinal: int) -> None:
        pass

    def elapsed_ms(self, start: int, stop: int) -> float:
        return 0.0


def _stub_device(name: str = "MI355X", ordinal: int = 0) -> R.MI355XDevice:
    import threading

    dev = object.__new__(R.MI355XDevice)
    dev.device, dev.ordinal, dev.lock, dev.failure = name, ordinal, threading.RLock(), None
    dev.stream, dev.inflight = 0x51, []
    dev.allocator = R.MI355XAllocator(dev)
    return dev


def _stub_program(dev: R.MI355XDevice) -> R.MI355XProgram:
    prog = object.__new__(R.MI355XProgram)
    prog.dev, prog.name, prog.function, prog.module = dev, "k", 0x99, 0
    prog.signature = KernelSignature("k", ("ptr", "i32"))
    return prog


def _buffer_on(dev, size=64):
    return R.MI355XBuffer(dev, R._Allocation(0x1000, size), size)


def test_a_failed_launch_is_sticky(monkeypatch):
    """A launch whose hipModuleLaunchKernel fails raises that error and is kept as the device's
    failure; every later launch, copy, transfer and synchronize raises from it, without reaching
    HIP (ops_dx12.py:196-198, :275-295; test_execution.py:128-165)."""
    stub = _StubHip()
    monkeypatch.setattr(R, "hip", stub)
    dev = _stub_device()
    prog, buf = _stub_program(dev), _buffer_on(dev)
    prog(buf, vals=(3,))  # a good launch first
    assert dev.failure is None and stub.calls.count("hipModuleLaunchKernel") == 1
    stub.armed.add("hipModuleLaunchKernel")
    with pytest.raises(RuntimeError, match="injected"):
        prog(buf, vals=(3,))
    assert isinstance(dev.failure, RuntimeError) and "injected" in str(dev.failure)
    before = len(stub.calls)
    later = [lambda: prog(buf, vals=(3,)), lambda: prog(buf, vals=(3,), wait=True),
             lambda: dev.allocator._copyin(buf, memoryview(bytes(8))),
             lambda: dev.allocator._copyout(memoryview(bytearray(8)), buf),
             lambda: dev.allocator._transfer(_buffer_on(dev), buf, 8, dev, dev),
             lambda: dev.synchronize()]
    for action in later:
        with pytest.raises(RuntimeError, match="submission/transfer failed") as info:
            action()
        assert info.value.__cause__ is dev.failure
    assert len(stub.calls) == before  # nothing after the failure reached HIP


@pytest.mark.parametrize("which", ["copyin", "copyout", "transfer"])
def test_a_failed_copy_is_sticky(monkeypatch, which):
    """A copy whose hipMemcpyAsync fails sets the failure too; later launches raise."""
    stub = _StubHip()
    monkeypatch.setattr(R, "hip", stub)
    dev = _stub_device()
    prog, buf = _stub_program(dev), _buffer_on(dev)
    stub.armed.add("hipMemcpyAsync")
    action = {"copyin": lambda: dev.allocator._copyin(buf, memoryview(bytes(8))),
              "copyout": lambda: dev.allocator._copyout(memoryview(bytearray(8)), buf),
              "transfer": lambda: dev.allocator._transfer(_buffer_on(dev), buf, 8, dev, dev)}[which]
    with pytest.raises(RuntimeError, match="injected"):
        action()
    assert dev.failure is not None
    assert all(name != "hipHostMalloc" for name in stub.calls)
    assert not stub._host  # staging memory of the failed copy was released
    with pytest.raises(RuntimeError, match="submission/transfer failed"):
        prog(buf, vals=(1,))
    with pytest.raises(RuntimeError, match="submission/transfer failed"):
        dev.synchronize()


def test_a_failed_cross_device_transfer_marks_both_devices(monkeypatch):
    stub = _StubHip()
    monkeypatch.setattr(R, "hip", stub)
    src, dst = _stub_device("MI355X", 0), _stub_device("MI355X:1", 1)
    stub.armed.add("hipMemcpyPeerAsync")
    with pytest.raises(RuntimeError, match="injected"):
        dst.allocator._transfer(_buffer_on(dst), _buffer_on(src), 16, src, dst)
    assert src.failure is dst.failure is not None
    for dev in (src, dst):
        with pytest.raises(RuntimeError, match="submission/transfer failed"):
            dev.synchronize()


def test_one_hip_runtime_whichever_is_opened_first():
    """The plugin's HIP binding and kernel library opened before torch is imported must leave one
    HIP runtime mapped once torch loads its own (torch's libraries ask for libamdhip64.so through
    their rpath, which the ROCm runtime's soname does not answer)."""
    import subprocess
    import sys
    from pathlib import Path

    pkg = Path(__file__).resolve().parents[1] / "tinygrad-dx12_amd"
    code = (f"import sys; sys.path.insert(0, {str(pkg)!r})\n"
            "from tinygrad_mi355x.runtime.support import hip\n"
            "hip.library()\n"
            "from tinygrad_mi355x.runtime import library\n"
            "library.load_library()\n"
            "import torch\n"
            "from tinygrad_mi355x.runtime import kernels\n"
            "print(len(hip._loaded_runtimes()))\n")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().splitlines()[-1] == "1"


def test_dump_src_prints_each_new_source_once(monkeypatch, capsys):
    """MI355X_DUMP_SRC=1 prints what the compiler compiles (the reference's DX12_DUMP_SHADERS),
    before invoking the toolchain, once per new source."""
    from tinygrad_mi355x.runtime.support import compiler_hip as CH

    comp = CH.MI355XCompiler("gfx950")
    src = MI355XRenderer("gfx950").render(KernelSpec("dumped", (BufferParam("x", torch.float32),),
                                                     body=("x[0] = 1.0f;",)))
    monkeypatch.setenv("MI355X_DUMP_SRC", "1")
    calls = []

    def fake_run(cmd, capture_output, text):
        calls.append(cmd)
        Path(cmd[-1]).write_bytes(b"\x7fELF-not-really")
        return subprocess.CompletedProcess(cmd, 0, "", "")

    monkeypatch.setattr(CH.subprocess, "run", fake_run)
    comp.compile(src)
    comp.compile(src)
    err = capsys.readouterr().err
    assert err.count("dumped") >= 1 and err.count(src) == 1 and len(calls) == 1
    monkeypatch.setenv("MI355X_DUMP_SRC", "0")
    comp2 = CH.MI355XCompiler("gfx950")
    comp2.compile(src)
    assert capsys.readouterr().err == ""


def test_profile_events_from_eager_graph_and_library_calls_with_stubbed_hip(monkeypatch):
    """With profiling on, an eager launch publishes a ProfileRangeEvent and a graph replay a
    ProfileGraphEvent with one entry per kernel over kernel_count + 1 signals, read from the
    events recorded around them (HIP stubbed: event i completes at 10 * i microseconds)."""
    import decimal

    from tinygrad_mi355x.runtime import profile

    times: dict[int, float] = {}
    counter = iter(range(1, 10_000))
    recorded = []

    class Stub:
        def __init__(self):
            self.now = 0.0

    stub = Stub()

    def event_create():
        e = next(counter)
        times[e] = 0.0
        return e

    def call(name, *args):
        if name in ("hipEventRecord", "hipEventRecordWithFlags"):
            stub.now += 0.01  # ms
            times[args[0]] = stub.now
            recorded.append((name, args[-1] if name == "hipEventRecordWithFlags" else None))
        return 0

    monkeypatch.setattr(profile.hip, "event_create", event_create)
    monkeypatch.setattr(profile.hip, "call", call)
    monkeypatch.setattr(profile.hip, "elapsed_ms", lambda a, b: times[b] - times[a])

    class Dev:
        device = "MI355X"
        stream = 7

    dev = Dev()
    profile.profile_events.clear()
    rng = profile.RangeTiming(dev, "k_eager")
    rng.end(dev)
    rng.publish()
    timing = profile.GraphTiming(dev, ["k0", "k1", "k2"])
    for e in timing.events:  # what a replay's event-record nodes do
        call("hipEventRecord", e, dev.stream)
    event = timing.publish()
    kinds = [type(e).__name__ for e in profile.profile_events]
    assert kinds == ["ProfileDeviceEvent", "ProfileRangeEvent", "ProfileGraphEvent"]
    r = profile.profile_events[1]
    assert r.name == "k_eager" and abs(r.en - r.st - decimal.Decimal("10.0")) < decimal.Decimal("1e-9")
    assert [e.name for e in event.ents] == ["k0", "k1", "k2"] and len(event.sigs) == 4
    assert [(e.st_id, e.en_id) for e in event.ents] == [(0, 1), (1, 2), (2, 3)]
    assert event.deps == [[], [0], [1]]
    assert [round(s, 9) for s in profile.kernel_seconds(event)] == [1e-5, 1e-5, 1e-5]


def test_profiled_graph_records_an_event_node_around_every_call(monkeypatch):
    """StreamGraph.profiled captures the calls once, with an event node before the first call,
    between calls and after the last (HIP stubbed: the capture-time calls are logged)."""
    from tinygrad_mi355x.runtime import graph as G

    log = []
    monkeypatch.setattr(G.hip, "capture_begin", lambda stream: log.append(("begin", stream)))
    monkeypatch.setattr(G.hip, "capture_end", lambda stream: log.append(("end", stream)) or 7)
    monkeypatch.setattr(G.hip, "graph_instantiate", lambda graph: 8)
    monkeypatch.setattr(G.hip, "capture_event", lambda stream, event: log.append(("event", event)))
    g = G.StreamGraph.profiled([lambda: log.append(("call", 0)), lambda: log.append(("call", 1))], 5, [11, 12, 13])
    assert log == [("begin", 5), ("event", 11), ("call", 0), ("event", 12), ("call", 1), ("event", 13), ("end", 5)]
    assert (g._graph, g._exec) == (7, 8)
    g._graph = g._exec = 0  # nothing real to destroy
    with pytest.raises(ValueError, match="one event more"):
        G.StreamGraph.profiled([lambda: None], 5, [1])
