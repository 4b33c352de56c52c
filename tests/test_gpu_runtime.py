"""GPU tests of the device plugin (ops_mi355x): allocator, transfers, compile + launch,
timing, argument errors, and the packed GEMV driven through plugin buffers and the C ABI.

Modelled on the reference's device tests (test/device/test_execution.py,
test_large_address.py, test_shared_transfer.py) for the parts one GPU can show.
"""

import ctypes

import numpy as np
import pytest
import torch

import packed_oracle as O
from tinygrad_mi355x.renderer.cstyle import BufferParam, KernelSpec
from tinygrad_mi355x.runtime import kernels as K
from tinygrad_mi355x.runtime import ops_mi355x as R

pytestmark = pytest.mark.gpu

SAXPY = KernelSpec("saxpy", (BufferParam("y", torch.float32, True), BufferParam("x", torch.float32)),
                   (("a", "f32"), ("n", "i32")),
                   ("const int i = gidx0 * 256 + lidx0;", "if (i < n) y[i] = a * x[i] + y[i];"))


@pytest.fixture(scope="module")
def device():
    d = R.get_device("MI355X")
    yield d
    d.synchronize()


def upload(dev, arr: np.ndarray) -> R.MI355XBuffer:
    buf = dev.allocator.alloc(arr.nbytes)
    dev.allocator._copyin(buf, memoryview(np.ascontiguousarray(arr)).cast("B"))
    return buf


def download(dev, buf, dtype, count) -> np.ndarray:
    out = np.empty(count, dtype)
    dev.allocator._copyout(memoryview(out).cast("B"), buf)
    return out


def test_device_identity(device):
    assert device.count() >= 1
    assert device.arch == "gfx950"
    assert device.renderer.compiler.arch == "gfx950"


def test_copy_round_trip_offsets_and_zero_fill(device):
    rng = np.random.default_rng(0)
    data = rng.integers(0, 256, 1 << 20, dtype=np.uint8)
    buf = upload(device, data)
    assert np.array_equal(download(device, buf, np.uint8, data.size), data)
    view = device.allocator._offset(buf, 4096, 12345)
    assert np.array_equal(download(device, view, np.uint8, 4096), data[12345:12345 + 4096])
    z = device.allocator._alloc(1000, R.BufferSpec(zero=True))
    assert not download(device, z, np.uint8, 1000).any()
    device.allocator.free(buf, buf.size)
    device.allocator.free(z, 1000)
    device.synchronize()
    device.allocator.free_cache()


def test_copyin_owns_the_callers_bytes(device):
    src = bytearray(b"\x11" * 4096)
    buf = device.allocator.alloc(4096)
    device.allocator._copyin(buf, memoryview(src))
    src[:] = b"\x22" * 4096  # mutate immediately: the upload must already own a copy
    assert (download(device, buf, np.uint8, 4096) == 0x11).all()


@pytest.mark.parametrize("shift", [-1000, 1000, 0])
def test_transfer_including_overlapping_views(device, shift):
    base = np.arange(16384, dtype=np.uint8) * 7
    buf = upload(device, base)
    src = device.allocator._offset(buf, 8192, 4096)
    dst = device.allocator._offset(buf, 8192, 4096 + shift)
    device.allocator._transfer(dst, src, 8192, device, device)
    want = base.copy()
    want[4096 + shift:4096 + shift + 8192] = base[4096:4096 + 8192]
    assert np.array_equal(download(device, buf, np.uint8, base.size), want)
    other = device.allocator.alloc(8192)
    device.allocator._transfer(other, src, 8192, device, device)
    assert np.array_equal(download(device, other, np.uint8, 8192), want[4096:4096 + 8192])


def test_compile_launch_and_timing(device):
    src = device.renderer.render(SAXPY)
    prog = device.runtime("saxpy", device.compiler.compile(src))
    n = 1_000_003
    rng = np.random.default_rng(1)
    x, y = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    bx, by = upload(device, x), upload(device, y)
    groups = (n + 255) // 256
    assert prog(by, bx, global_size=(groups, 1, 1), local_size=(256, 1, 1), vals=(2.5, n)) is None
    seconds = prog(by, bx, global_size=(groups, 1, 1), local_size=(256, 1, 1), vals=(-1.0, n), wait=True)
    assert isinstance(seconds, float) and 0 < seconds < 1
    got = download(device, by, np.float32, n)
    want = -1.0 * x.astype(np.float64) + (2.5 * x.astype(np.float64) + y)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)  # the device may contract a*x+y to an FMA
    assert prog(by, bx, global_size=(0, 1, 1), vals=(1.0, n), wait=True) == 0.0
    with pytest.raises(ValueError):
        prog(by, vals=(1.0, n))
    with pytest.raises(ValueError):
        prog(by, bx, vals=(1.0,))
    other = R.MI355XDevice("MI355X")  # a second device object: its buffers are foreign here
    with pytest.raises(ValueError):
        prog(by, other.allocator.alloc(64), vals=(1.0, n))


def test_packed_gemv_through_plugin_buffers(device):
    """The standalone chain: plugin allocations + the C-ABI GEMV on the device's stream."""
    rng = np.random.default_rng(2)
    n, k = 1024, 4096
    codes = rng.integers(0, 16, (n, k)).astype(np.uint8)
    e = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.uint8)
    xb = O.bf16_round(rng.standard_normal(k).astype(np.float32))  # bf16 bit patterns
    x = O.bf16_to_f32(xb)
    data = O.pack_codes(codes, 4)
    bw, bs, bx = upload(device, data), upload(device, e), upload(device, xb)
    by = device.allocator.alloc(n * 4)
    lib = K.load_library()
    K.check("tgm_gemv", lib.tgm_gemv(bw.address, K.FORMAT_IDS["fp4_e2m1"], n, k, bs.address,
                                     K.DTYPE_IDS[torch.float8_e8m0fnu], 32, bx.address, K.DTYPE_IDS[torch.bfloat16],
                                     1, k, by.address, K.DTYPE_IDS[torch.float32], n, ctypes.c_void_p(device.stream)))
    device.synchronize()
    got = download(device, by, np.float32, n)
    deq = O.dequant_f64(data, "fp4_e2m1", (n, k), O.e8m0_decode(e), 32)
    want = deq @ x.astype(np.float64)
    assert O.max_rel_err(got, want) <= 1e-4  # fp32 output: only the summation order differs


def test_graph_replays_program_sequence(device):
    """MI355XGraph (the reference's graph runner, runtime/graph/dx12.py:49-253): a sequence of
    program calls replayed as one HIP graph equals the eager sequence, replay after replay with
    eager work in between; changed scalars re-record; wait=True returns GPU seconds."""
    from tinygrad_mi355x.runtime.graph import MI355XGraph

    src = device.renderer.render(SAXPY)
    prog = device.runtime("saxpy", device.compiler.compile(src))
    n = 100_003
    rng = np.random.default_rng(3)
    x, y0 = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    bx, by = upload(device, x), upload(device, y0)
    groups = ((n + 255) // 256, 1, 1)
    calls = [(prog, (by, bx), groups, (256, 1, 1), (0.5, n)), (prog, (by, bx), groups, (256, 1, 1), (-2.0, n))]
    graph = MI355XGraph(calls)
    want = y0.astype(np.float64)
    for replay in range(4):
        seconds = graph(wait=(replay == 3))
        want = want + 0.5 * x - 2.0 * x
        if replay == 1:  # eager work between replays, ordered on the same stream
            prog(by, bx, global_size=groups, local_size=(256, 1, 1), vals=(1.0, n))
            want = want + x
        device.synchronize()
        np.testing.assert_allclose(download(device, by, np.float32, n), want, rtol=1e-5, atol=1e-5)
    assert isinstance(seconds, float) and 0 < seconds < 1
    graph({1: ((by, bx), groups, (256, 1, 1), (3.0, n))})  # new scalar: the graph is recorded again
    device.synchronize()
    want = want + 0.5 * x + 3.0 * x
    np.testing.assert_allclose(download(device, by, np.float32, n), want, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        graph({0: ((by,), groups, (256, 1, 1), (1.0, n))})  # wrong buffer count, rejected before capture
    graph.close()


def test_profiling_publishes_per_kernel_times(device):
    """Under profiling: an eager launch publishes a ProfileRangeEvent, a library program on
    plugin buffers one too, and each replay of a three-kernel graph a ProfileGraphEvent whose
    three entries cover four signals recorded as graph nodes (the reference's kernel_count + 1
    timestamp queries).  The kernels' times are positive and in launch order, the larger kernel
    takes longer than the small one after it, and the graph still computes what the eager
    sequence does."""
    from tinygrad_mi355x.runtime import profile
    from tinygrad_mi355x.runtime.graph import MI355XGraph

    src = device.renderer.render(SAXPY)
    prog = device.runtime("saxpy", device.compiler.compile(src))
    n_big, n = 8_000_000, 100_003
    rng = np.random.default_rng(5)
    x, y0 = rng.standard_normal(n_big).astype(np.float32), rng.standard_normal(n_big).astype(np.float32)
    bx, by = upload(device, x), upload(device, y0)
    small, big = (((n + 255) // 256, 1, 1), ((n_big + 255) // 256, 1, 1))
    profile.set_enabled(True)
    try:
        profile.profile_events.clear()
        print("profiled eager launch", flush=True)
        prog(by, bx, global_size=small, local_size=(256, 1, 1), vals=(1.0, n))
        device.synchronize()
        ranges = [e for e in profile.profile_events if type(e).__name__ == "ProfileRangeEvent"]
        assert len(ranges) == 1 and ranges[0].name == "saxpy" and ranges[0].en > ranges[0].st
        print("profiled three-kernel graph", flush=True)
        calls = [(prog, (by, bx), small, (256, 1, 1), (0.5, n)), (prog, (by, bx), big, (256, 1, 1), (-2.0, n_big)),
                 (prog, (by, bx), small, (256, 1, 1), (0.25, n))]
        graph = MI355XGraph(calls)
        for _ in range(3):
            graph()
        device.synchronize()
        events = [e for e in profile.profile_events if type(e).__name__ == "ProfileGraphEvent"]
        assert len(events) == 3
        for ev in events:
            assert [e.name for e in ev.ents] == ["saxpy"] * 3 and len(ev.sigs) == 4
            assert all(a < b for a, b in zip(ev.sigs, ev.sigs[1:]))
            secs = profile.kernel_seconds(ev)
            # the first interval also holds the replay's start; the 80x larger middle kernel
            # outlasts the last
            assert all(0 < s < 0.1 for s in secs) and secs[1] > secs[2]
        assert events[1].sigs[0] > events[0].sigs[-1]  # replays in stream order
        graph.close()
    finally:
        profile.set_enabled(False)
    want = y0.astype(np.float64)
    want[:n] += 1.0 * x[:n]
    for _ in range(3):
        want[:n] += 0.5 * x[:n]
        want += -2.0 * x
        want[:n] += 0.25 * x[:n]
    np.testing.assert_allclose(download(device, by, np.float32, n_big), want, rtol=1e-4, atol=1e-4)
