"""MI355X device plugin: Device, Allocator, Buffer and Program over the HIP runtime.

Counterpart of the reference's DX12 runtime (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/runtime/ops_dx12.py:150-744), with the same surface and contracts:

* ``MI355XDevice(device)`` -- ``.renderer``, ``.runtime(name, lib)``, ``.synchronize(timeout)``,
  ``.count()``; a per-device ``RLock`` around submission (ops_dx12.py:155) and a sticky
  failure: a HIP call that fails while enqueueing a launch, copy or transfer is kept as
  ``dev.failure``, and every later launch, copy, transfer and synchronize raises
  ``RuntimeError("MI355X submission/transfer failed")`` from it (:197-198, :275-295); a
  failed cross-device transfer marks both devices.
* ``MI355XAllocator(dev)`` -- ``_alloc`` rejects ``external_ptr`` and zero-fills on
  ``zero`` (:440-447); ``_copyin`` owns the caller's bytes before returning and is
  asynchronous (:455-461); ``_copyout`` blocks (:463-470); ``_offset`` is bounds checked
  and raises ``ValueError`` (:449-453); ``free`` defers reuse until the GPU is done with
  the storage (:429-438); ``_transfer`` copies between views, including overlapping
  views of one allocation (:479-499).
* ``MI355XProgram(dev, name, lib)`` -- ``__call__(*bufs, global_size, local_size, vals,
  wait, timeout)`` with group-count semantics, zero work -> ``0.0 if wait else None``,
  and ``ValueError`` on buffer, device or scalar count mismatch (:659-744).

What changes is the machinery: one HIP stream per device instead of a D3D12 queue and
fence, ``hipMalloc`` allocations instead of placed resources, pinned staging buffers
instead of UPLOAD/READBACK heaps, HIP events instead of fence values, and
``hipModuleLaunchKernel`` with a packed kernarg buffer instead of root signatures and
descriptor tables.  No stream is created at a non-default priority.
"""

from __future__ import annotations

import contextlib
import ctypes
import struct
import threading
import time
from dataclasses import dataclass, field
from typing import Callable

from tinygrad_mi355x.compat import DEVICE
from tinygrad_mi355x.renderer.cstyle import MI355XRenderer
from tinygrad_mi355x.runtime import profile
from tinygrad_mi355x.runtime.support import hip
from tinygrad_mi355x.runtime.support.compiler_hip import CompileError, unpack_object

__all__ = ["MI355XDevice", "MI355XAllocator", "MI355XBuffer", "MI355XProgram", "BufferSpec", "CompileError",
           "get_device"]

DEFAULT_TIMEOUT_MS = 120_000


@dataclass(frozen=True)
class BufferSpec:
    """Allocation options (the fields of tinygrad's BufferSpec this device honours)."""

    zero: bool = False
    host: bool = False
    external_ptr: int | None = None
    nolru: bool = False


@dataclass
class _Allocation:
    """One hipMalloc (or pinned host) allocation and the completion events of work that uses it."""

    ptr: int
    size: int
    host: bool = False
    uses: list = field(default_factory=list)  # HIP events recorded after work that touched it
    freed: bool = False


class MI355XBuffer:
    """A byte view ``[offset, offset + size)`` of one allocation."""

    def __init__(self, dev: "MI355XDevice", owner: _Allocation, size: int, offset: int = 0) -> None:
        self.dev, self.owner, self.size, self.offset = dev, owner, size, offset

    @property
    def address(self) -> int:
        return self.owner.ptr + self.offset

    def __repr__(self) -> str:
        return f"<MI355XBuffer {self.dev.device} 0x{self.address:x} size={self.size}>"


class MI355XAllocator:
    """Device memory with deferred reuse, pinned staging copies and an LRU free cache."""

    def __init__(self, dev: "MI355XDevice") -> None:
        self.dev = dev
        self.cache: dict[tuple[int, BufferSpec], list[MI355XBuffer]] = {}
        self.retired: list[tuple[MI355XBuffer, int, BufferSpec]] = []

    # ---- tinygrad LRUAllocator-style entry points ----
    def alloc(self, size: int, options: BufferSpec | None = None) -> MI355XBuffer:
        options = options or BufferSpec()
        with self.dev.lock:
            self._collect()
            cached = self.cache.get((size, options))
            if cached and not options.zero:
                return cached.pop()
        return self._alloc(size, options)

    def free(self, buf: MI355XBuffer, size: int, options: BufferSpec | None = None) -> None:
        """Keep storage out of the reusable cache until the GPU work using it has completed."""
        with self.dev.lock:
            self.retired.append((buf, size, options or BufferSpec()))
            self._collect()

    def free_cache(self) -> None:
        """Release completed cached storage; storage still referenced by GPU work is retained."""
        with self.dev.lock:
            self._collect()
            for bufs in self.cache.values():
                for buf in bufs:
                    self._free(buf)
            self.cache.clear()

    def _collect(self) -> None:
        pending = []
        for buf, size, options in self.retired:
            if self.dev.idle(buf.owner):
                if options.nolru:
                    self._free(buf)
                else:
                    self.cache.setdefault((size, options), []).append(buf)
            else:
                pending.append((buf, size, options))
        self.retired = pending

    # ---- device-specific primitives ----
    def _alloc(self, size: int, options: BufferSpec) -> MI355XBuffer:
        """Allocate ``size`` bytes; external pointers are not accepted as allocations."""
        if options.external_ptr is not None:
            raise ValueError("MI355X external_ptr is not supported: allocations must come from hipMalloc")
        if size < 0:
            raise ValueError("MI355X allocation size must be nonnegative")
        with self.dev.lock:
            self.dev.select()
            ptr = hip.host_malloc(size) if options.host else hip.malloc(size)
        buf = MI355XBuffer(self.dev, _Allocation(ptr, size, host=options.host), size)
        if options.zero and size:
            self._copyin(buf, memoryview(bytes(size)))
        return buf

    def _free(self, buf: MI355XBuffer, options: BufferSpec | None = None) -> None:
        owner = buf.owner
        if owner.freed:
            return
        with self.dev.lock:
            self.dev.select()
            self.dev.wait_owner(owner)
            hip.call("hipHostFree" if owner.host else "hipFree", owner.ptr)
            owner.freed = True

    def _offset(self, buf: MI355XBuffer, size: int, offset: int) -> MI355XBuffer:
        """A bounds-checked byte view that keeps the original allocation alive."""
        if offset < 0 or size < 0 or offset + size > buf.size:
            raise ValueError("MI355X view outside allocation")
        return MI355XBuffer(self.dev, buf.owner, size, buf.offset + offset)

    def _copyin(self, dest: MI355XBuffer, src: memoryview) -> None:
        """Copy host bytes to the device; the bytes are owned (staged) before this returns."""
        nbytes = src.nbytes
        if nbytes > dest.size:
            raise ValueError("MI355X upload exceeds view size")
        if nbytes == 0:
            return
        with self.dev.lock, self.dev.submitting():
            self.dev.select()
            staging = hip.host_malloc(nbytes)
            ctypes.memmove(staging, (ctypes.c_char * nbytes).from_buffer_copy(src.cast("B")), nbytes)
            try:
                hip.call("hipMemcpyAsync", dest.address, staging, nbytes, hip.H2D, self.dev.stream)
            except RuntimeError:
                hip.call("hipHostFree", staging)
                raise
            self.dev.submitted((dest.owner,), lambda: hip.call("hipHostFree", staging))

    def _copyout(self, dest: memoryview, src: MI355XBuffer) -> None:
        """Copy device bytes to host memory; waits for the copy."""
        nbytes = dest.nbytes
        if nbytes > src.size:
            raise ValueError("MI355X readback exceeds view size")
        if nbytes == 0:
            return
        with self.dev.lock:
            with self.dev.submitting():
                self.dev.select()
                staging = hip.host_malloc(nbytes)
            try:
                with self.dev.submitting():
                    hip.call("hipMemcpyAsync", staging, src.address, nbytes, hip.D2H, self.dev.stream)
                    event = self.dev.submitted((src.owner,))
                self.dev.wait_event(event)
                ctypes.memmove((ctypes.c_char * nbytes).from_buffer(dest.cast("B")), staging, nbytes)
            finally:
                hip.call("hipHostFree", staging)

    def _transfer(self, dest: MI355XBuffer, src: MI355XBuffer, sz: int, src_dev: "MI355XDevice",
                  dest_dev: "MI355XDevice") -> None:
        """Ordered device-to-device copy of ``sz`` bytes, including overlapping views."""
        if sz < 0 or sz > src.size or sz > dest.size:
            raise ValueError("MI355X transfer exceeds view size")
        if sz == 0:
            return
        if src_dev is dest_dev:
            if src.owner is dest.owner and src.offset == dest.offset:
                return
            with self.dev.lock, self.dev.submitting():
                self.dev.select()
                overlap = (src.owner is dest.owner and src.offset < dest.offset + sz and dest.offset < src.offset + sz)
                if overlap:
                    tmp = self._alloc(sz, BufferSpec())
                    hip.call("hipMemcpyAsync", tmp.address, src.address, sz, hip.D2D, self.dev.stream)
                    hip.call("hipMemcpyAsync", dest.address, tmp.address, sz, hip.D2D, self.dev.stream)
                    self.dev.submitted((src.owner, dest.owner, tmp.owner))
                    self.free(tmp, sz, BufferSpec(nolru=True))
                else:
                    hip.call("hipMemcpyAsync", dest.address, src.address, sz, hip.D2D, self.dev.stream)
                    self.dev.submitted((src.owner, dest.owner))
            return
        # Cross-device: order after the source device's work, copy on the destination's stream.
        src_dev.synchronize()
        with dest_dev.lock, dest_dev.submitting(src_dev):
            dest_dev.select()
            hip.call("hipMemcpyPeerAsync", dest.address, dest_dev.ordinal, src.address, src_dev.ordinal, sz,
                     dest_dev.stream)
            dest_dev.submitted((dest.owner,))


class MI355XProgram:
    """One kernel of a compiled object, launched with group-count semantics."""

    def __init__(self, dev: "MI355XDevice", name: str, lib: bytes) -> None:
        self.dev, self.name = dev, name
        self.source, self.signature, code = unpack_object(lib)
        if self.signature.name != name:
            raise ValueError(f"MI355X program {name!r} does not match compiled kernel {self.signature.name!r}")
        with dev.lock:
            dev.select()
            self.module, self._image = hip.module_load(code)
            self.function = hip.module_function(self.module, name)

    def _kernargs(self, bufs, vals) -> bytes:
        out = bytearray()
        it_b, it_v = iter(bufs), iter(vals)
        fmt = {"i32": "<i", "u32": "<I", "i64": "<q", "u64": "<Q", "f32": "<f", "f64": "<d"}
        for kind in self.signature.params:
            if kind == "ptr":
                data, align = struct.pack("<Q", next(it_b).address), 8
            else:
                data = struct.pack(fmt[kind], next(it_v))
                align = len(data)
            out += b"\0" * (-len(out) % align)
            out += data
        return bytes(out)

    def validate(self, bufs, global_size, local_size, vals) -> tuple[tuple[int, int, int], tuple[int, int, int]]:
        """Check a launch's arguments (ValueError on any mismatch); returns the launch sizes."""
        global_size = tuple(global_size or (1, 1, 1))
        local_size = tuple(local_size or (1, 1, 1))
        limits = MI355XRenderer.global_max
        if len(global_size) != 3 or any(x < 0 or x > lim for x, lim in zip(global_size, limits)):
            raise ValueError("invalid MI355X dispatch dimensions")
        if len(local_size) != 3 or any(x < 1 for x in local_size) or local_size[0] * local_size[1] * local_size[2] > 1024:
            raise ValueError("invalid MI355X workgroup dimensions")
        if len(bufs) != self.signature.buffers or any(not isinstance(b, MI355XBuffer) or b.dev is not self.dev
                                                      for b in bufs):
            raise ValueError("MI355X buffer device/signature mismatch")
        if 0 not in global_size and len(vals) != self.signature.scalars:
            raise ValueError("MI355X scalar argument count mismatch")
        return global_size, local_size

    def enqueue(self, bufs, global_size, local_size, vals) -> None:
        """Launch validated arguments on the device stream (the caller holds the device lock)."""
        if 0 in global_size:
            return
        hip.launch(self.function, tuple(global_size), tuple(local_size), self._kernargs(bufs, vals), self.dev.stream)

    def __call__(self, *bufs: MI355XBuffer, global_size: tuple[int, int, int] = (1, 1, 1),
                 local_size: tuple[int, int, int] = (1, 1, 1), vals: tuple[int | float, ...] = (), wait: bool = False,
                 timeout: int | None = None) -> float | None:
        """Launch ``global_size`` workgroups of ``local_size`` work-items; seconds when ``wait``."""
        global_size, local_size = self.validate(bufs, global_size, local_size, vals)
        if 0 in global_size:
            return 0.0 if wait else None
        with self.dev.lock, self.dev.submitting():
            self.dev.select()
            # timing events belong to this call only (the device retires and destroys its own)
            start, stop = (hip.event_create(), hip.event_create()) if wait else (0, 0)
            ranged = profile.RangeTiming(self.dev, self.name) if profile.enabled() else None
            if wait:
                hip.call("hipEventRecord", start, self.dev.stream)
            self.enqueue(bufs, global_size, local_size, vals)
            if wait:
                hip.call("hipEventRecord", stop, self.dev.stream)
            if ranged is not None:
                ranged.end(self.dev)
            self.dev.submitted(tuple(b.owner for b in bufs), ranged.publish if ranged is not None else None)
        if not wait:
            return None
        try:
            self.dev.wait_event(stop, timeout, owned=True)
            return hip.elapsed_ms(start, stop) / 1e3
        finally:
            hip.call("hipEventDestroy", start)
            hip.call("hipEventDestroy", stop)

    def __del__(self) -> None:
        module = getattr(self, "module", 0)
        if module:
            try:
                hip.library().hipModuleUnload(module)
            except Exception:  # noqa: BLE001 -- interpreter shutdown
                pass


class MI355XDevice:
    """One MI355X: its HIP stream, allocator, renderer/compiler and submission lock."""

    wait_timeout_ms = DEFAULT_TIMEOUT_MS

    def __init__(self, device: str = DEVICE) -> None:
        """Open device ``MI355X`` or ``MI355X:<ordinal>``; raises when it does not exist."""
        self.device = device
        self.ordinal = int(device.split(":")[1]) if ":" in device else 0
        self.lock = threading.RLock()
        self.failure: BaseException | None = None
        hip.init()
        count = hip.device_count()
        if not 0 <= self.ordinal < count:
            raise RuntimeError(f"{device}: no such HIP device ({count} visible)")
        self.select()
        self.stream = hip.stream_create()
        self.inflight: list[tuple[int, tuple[_Allocation, ...], Callable[[], None] | None]] = []
        self.arch = _arch_of(self.ordinal)
        self._renderer = MI355XRenderer(self.arch)
        self.compiler = self._renderer.compiler
        self.allocator = MI355XAllocator(self)

    @property
    def renderer(self) -> MI355XRenderer:
        return self._renderer

    def count(self) -> int:
        """Number of visible HIP devices."""
        return hip.device_count()

    def runtime(self, name: str, lib: bytes) -> MI355XProgram:
        """Create a program for kernel ``name`` of a compiled object on this device."""
        return MI355XProgram(self, name, lib)

    def select(self) -> None:
        hip.set_device(self.ordinal)

    def check_failure(self) -> None:
        """Re-raise a failed submission: the stream's contents are unknown after it."""
        if self.failure is not None:
            raise RuntimeError(f"{self.device} submission/transfer failed") from self.failure

    @contextlib.contextmanager
    def submitting(self, *others: "MI355XDevice"):
        """Guard one enqueue: refuse it after an earlier failure, and keep a HIP failure raised
        inside it as this device's (and ``others``') sticky failure."""
        self.check_failure()
        for dev in others:
            dev.check_failure()
        try:
            yield
        except RuntimeError as exc:
            for dev in (self, *others):
                if dev.failure is None:
                    dev.failure = exc
            raise

    def submitted(self, owners: tuple[_Allocation, ...], callback: Callable[[], None] | None = None) -> int:
        """Record a completion event after the work just enqueued; owners stay busy until it fires."""
        self.check_failure()
        event = hip.event_create()
        hip.call("hipEventRecord", event, self.stream)
        for owner in owners:
            owner.uses.append(event)
        self.inflight.append((event, owners, callback))
        return event

    def retire(self) -> None:
        """Run callbacks and release bookkeeping of completed work."""
        with self.lock:
            pending = []
            for event, owners, callback in self.inflight:
                if hip.query("hipEventQuery", event):
                    for owner in owners:
                        if event in owner.uses:
                            owner.uses.remove(event)
                    if callback is not None:
                        callback()
                    hip.call("hipEventDestroy", event)
                else:
                    pending.append((event, owners, callback))
            self.inflight = pending

    def idle(self, owner: _Allocation) -> bool:
        self.retire()
        return not owner.uses

    def wait_event(self, event: int, timeout: int | None = None, owned: bool = False) -> None:
        """Wait (without holding the lock) until ``event`` completes, or time out.

        ``event`` is one of the device's in-flight events (returned by ``submitted``), which
        the device destroys once retired -- a retired event counts as complete -- or, with
        ``owned``, an event the caller created and destroys itself.
        """
        deadline = time.monotonic() + (timeout or self.wait_timeout_ms) / 1000
        delay = 1e-5
        while True:
            with self.lock:
                if not owned and all(e != event for e, _, _ in self.inflight):
                    break
                if hip.query("hipEventQuery", event):
                    break
            if time.monotonic() > deadline:
                raise RuntimeError(f"{self.device} wait timed out")
            time.sleep(delay)
            delay = min(delay * 2, 1e-3)
        self.retire()

    def wait_owner(self, owner: _Allocation) -> None:
        for event in list(owner.uses):
            self.wait_event(event)

    def synchronize(self, timeout: int | None = None) -> None:
        """Wait for all work submitted to this device."""
        with self.lock:
            self.check_failure()
            self.select()
            event = self.submitted(())
        self.wait_event(event, timeout)


def _arch_of(ordinal: int) -> str:
    """The device's architecture from the kernel library (hipGetDeviceProperties' gcnArchName);
    gfx950, the only target the library is built for, when the library is not built."""
    from tinygrad_mi355x.runtime import library

    try:
        return library.device_arch(ordinal)
    except (OSError, RuntimeError) as error:
        if "not built" in str(error):
            return "gfx950"
        raise


_devices: dict[str, MI355XDevice] = {}
_devices_lock = threading.Lock()


def get_device(device: str = DEVICE) -> MI355XDevice:
    """The process-wide device object for ``device`` (standalone use, without tinygrad's Device registry)."""
    with _devices_lock:
        if device not in _devices:
            _devices[device] = MI355XDevice(device)
        return _devices[device]

