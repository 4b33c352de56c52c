"""Running a schedule (a LINEAR of CALLs) on one MI355X.

The reference leaves execution to tinygrad: each CALL becomes a compiled program launched through
``DX12Program.__call__`` with the CALL's buffers (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/runtime/ops_dx12.py:659-744), and native matrix CALLs carry a prebuilt
PROGRAM (codegen/linalg.py:37-58, codegen/matmul.py:206-218).  ``run_linear`` is that loop for
the schedules of ``uop/ops.py``:

* a CALL whose body is a kernel SINK is linearized (``uop/linearize.py``), rendered by the
  device's renderer, compiled by its compiler (both cache by source) and launched as an
  ``MI355XProgram`` with the CALL's buffers in the kernel's PARAM slot order and the values of
  its DEFINE_VARs;
* a CALL whose body is a PROGRAM (a ``MatrixProgram`` of the kernel library, as
  ``codegen/uop_matmul.py`` makes them) is launched with its (out, a, b) buffers;
* a BUFFER the caller does not bind is allocated from the device's allocator on first use.

Launches go to the device stream in order under the device lock, as every plugin launch does; the
returned map holds every buffer of the schedule, so results are read with the allocator's
``_copyout``.  ``LinearGraph`` captures a whole schedule into one HIP graph and replays it.
"""

from __future__ import annotations

from dataclasses import dataclass

from tinygrad_mi355x.codegen.program import MatrixProgram
from tinygrad_mi355x.runtime import profile
from tinygrad_mi355x.uop.linearize import LinearKernel, linearize
from tinygrad_mi355x.uop.ops import FP8_DTYPES, Ops, UOp, dtypes


@dataclass(frozen=True)
class CompiledKernel:
    listing: LinearKernel
    source: str
    program: object  # MI355XProgram


def compile_kernel(dev, sink: UOp) -> CompiledKernel:
    """Linearize, render and compile ``sink`` for ``dev`` (cached per device by kernel)."""
    cache = dev.__dict__.setdefault("_uop_kernels", {})
    found = cache.get(sink)
    if found is not None:
        return found
    listing = linearize(sink)
    source = dev.renderer.render(listing)
    program = dev.runtime(listing.name, dev.compiler.compile(source))
    cache[sink] = compiled = CompiledKernel(listing, source, program)
    return compiled


def _nbytes(u: UOp) -> int:
    return u.max_numel() * u.dtype.itemsize


@dataclass(frozen=True)
class Launch:
    """One resolved launch of a schedule: a library program with its (out, a[, b]) buffers, or a
    compiled kernel with its buffers, launch sizes and scalar values."""

    program: object
    bufs: tuple
    global_size: tuple[int, int, int] = (1, 1, 1)
    local_size: tuple[int, int, int] = (1, 1, 1)
    vals: tuple = ()

    @property
    def native(self) -> bool:
        return isinstance(self.program, MatrixProgram)

    def run(self) -> None:
        """Launch eagerly (under the device lock, recorded for the allocator's deferred frees)."""
        if self.native:
            self.program(*self.bufs)
        else:
            self.program(*self.bufs, global_size=self.global_size, local_size=self.local_size, vals=self.vals)

    def enqueue(self, stream: int) -> None:
        """Put the launch on ``stream`` with no locking or bookkeeping (stream capture)."""
        if self.native:
            out, a, *b = self.bufs
            self.program.launch(out.address, a.address, b[0].address if b else 0, stream)
        else:
            self.program.enqueue(self.bufs, self.global_size, self.local_size, self.vals)


def plan(dev, linear: UOp, buffers: dict | None = None, var_vals: dict[str, int] | None = None
         ) -> tuple[list[Launch], dict]:
    """Resolve every CALL of ``linear`` to a ``Launch``: kernels compiled, arguments checked,
    unbound BUFFERs allocated.  Returns the launches and the BUFFER -> MI355XBuffer map."""
    if linear.op is not Ops.LINEAR:
        raise ValueError("run_linear takes a LINEAR of CALLs")
    bound = dict(buffers or {})
    var_vals = var_vals or {}

    def buf(u: UOp):
        if u.op is not Ops.BUFFER:
            raise ValueError(f"a CALL argument must be a BUFFER, not {u.op.name}")
        got = bound.get(u)
        if got is None:
            got = bound[u] = dev.allocator.alloc(max(_nbytes(u), 1))
        elif got.size < _nbytes(u):
            raise ValueError("a bound buffer is smaller than its BUFFER")
        return got

    launches = []
    for call in linear.src:
        if call.op is not Ops.CALL:
            raise ValueError(f"LINEAR holds CALLs, not {call.op.name}")
        body, args = call.src[0], call.src[1:]
        if body.op is Ops.PROGRAM:
            prog = body.arg
            if not isinstance(prog, MatrixProgram) or len(args) not in (2, 3):
                raise ValueError("a PROGRAM call takes a library program and its (out, a[, b]) buffers")
            bufs = tuple(buf(a) for a in args)
            if any(b.dev is not dev for b in bufs):
                raise ValueError("MI355X buffer device/signature mismatch")
            # the library kernel reads and writes the extents its program records, which the
            # BUFFER UOps' own sizes need not cover
            prog.check_slots(tuple(b.size for b in bufs))
            launches.append(Launch(prog, bufs))
            continue
        if body.op is not Ops.SINK:
            raise ValueError(f"a CALL body is a SINK or a PROGRAM, not {body.op.name}")
        kernel = compile_kernel(dev, body)
        bufs = []
        for p in kernel.listing.params:
            if p.arg.slot + 1 >= len(call.src):
                raise ValueError(f"kernel {kernel.listing.name}: no argument for slot {p.arg.slot}")
            b = buf(args[p.arg.slot])
            arg_dt = args[p.arg.slot].dtype
            # an FP8 buffer binds a uint8 parameter: copies move FP8 elements as bytes
            same = arg_dt == p.dtype or (p.dtype == dtypes.uint8 and arg_dt in FP8_DTYPES)
            if b.size < _nbytes(p) or not same:
                raise ValueError(f"kernel {kernel.listing.name}: argument for slot {p.arg.slot} does not match")
            bufs.append(b)
        vals = tuple(int(var_vals[v.arg[0]]) for v in kernel.listing.variables)
        for v, x in zip(kernel.listing.variables, vals):
            if not v.arg[1] <= x <= v.arg[2]:
                raise ValueError(f"variable {v.arg[0]} = {x} is outside [{v.arg[1]}, {v.arg[2]}]")
        launch = Launch(kernel.program, tuple(bufs), kernel.listing.global_size, kernel.listing.local_size, vals)
        kernel.program.validate(launch.bufs, launch.global_size, launch.local_size, launch.vals)
        launches.append(launch)
    return launches, bound


def run_linear(dev, linear: UOp, buffers: dict | None = None, var_vals: dict[str, int] | None = None,
               wait: bool = False) -> dict:
    """Launch every CALL of ``linear`` in order on ``dev``; returns the BUFFER -> MI355XBuffer map
    (the caller's bindings plus what was allocated here).  With ``wait`` the device is
    synchronised before returning."""
    launches, bound = plan(dev, linear, buffers, var_vals)
    for launch in launches:
        launch.run()
    if wait:
        dev.synchronize()
    return bound


class LinearGraph:
    """A schedule captured once into a HIP graph and replayed with one launch (the reference's
    graph runner, runtime/graph/dx12.py:49-253, for whole schedules): kernels are compiled and
    buffers resolved before capture; every replay reads the buffers' current contents."""

    def __init__(self, dev, linear: UOp, buffers: dict | None = None, var_vals: dict[str, int] | None = None):
        from tinygrad_mi355x.runtime.graph import StreamGraph

        self.dev = dev
        self.launches, self.buffers = plan(dev, linear, buffers, var_vals)
        if not self.launches:
            raise ValueError("an empty schedule has nothing to capture")
        with dev.lock:
            dev.select()
            # under profiling: a timestamp node before the first kernel and after each
            self.timing = profile.GraphTiming(dev, [la.program.name for la in self.launches]) \
                if profile.enabled() else None

            def record() -> None:
                for launch in self.launches:
                    launch.enqueue(dev.stream)

            if self.timing is None:
                self.graph = StreamGraph(record, dev.stream)
            else:
                one = [lambda la=la: la.enqueue(dev.stream) for la in self.launches]
                self.graph = StreamGraph.profiled(one, dev.stream, self.timing.events)
        self.owners = tuple({id(b.owner): b.owner for la in self.launches for b in la.bufs}.values())

    def __call__(self, wait: bool = False) -> float | None:
        """Replay once (asynchronously); GPU seconds when ``wait``.  A graph captured under
        profiling waits for each replay and publishes its per-kernel times."""
        with self.dev.lock, self.dev.submitting():
            self.dev.select()
            seconds = self.graph(wait=wait or self.timing is not None)
            self.dev.submitted(self.owners)
            if self.timing is not None:
                self.timing.publish()
        return seconds if wait else None

    def close(self) -> None:
        self.graph.close()
        if self.timing is not None:
            self.timing.close()
            self.timing = None
