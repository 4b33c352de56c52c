"""HIP graph replay of recorded launch sequences.

The reference records a tinygrad kernel sequence into D3D12 command lists with patchable
descriptors and root constants, keeps a ring of three replay slots fenced by the queue, and
returns GPU seconds when asked to wait (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/runtime/graph/dx12.py:49-253).  On HIP the recording is stream capture and
the replay object is a hipGraphExec:

* ``StreamGraph`` captures whatever a callable launches on a stream (any mix of this
  package's kernels, C-ABI calls and plugin programs) and replays it with one
  ``hipGraphLaunch``.  Kernel arguments are baked in at capture time, so state that changes
  between replays (positions, tokens) lives in device memory.
* ``MI355XGraph`` is the plugin-level runner: a fixed list of ``MI355XProgram`` calls on one
  device.  A replay whose buffers, scalars or launch sizes differ from the recorded ones
  re-records the graph (the reference patches descriptors instead, dx12.py:180-248); a
  replay with the same arguments relaunches the graph as it is.

Replays are ordered on the stream like any other work, so a graph needs no ring of slots:
the GPU runs replay n + 1 after replay n.  Captured work must not allocate, synchronise or
issue memsets; the kernels of this package do none of those.

Under profiling (``runtime/profile.py``) a graph is captured with a timestamp event before its
first kernel and after each kernel, as graph nodes, and every replay waits for completion and
publishes a ``ProfileGraphEvent`` of per-kernel times (the reference's ``kernel_count + 1``
queries, runtime/graph/dx12.py:224, :249-253).
"""

from __future__ import annotations

import threading
from typing import Callable, Sequence

from tinygrad_mi355x.runtime import profile
from tinygrad_mi355x.runtime.support import hip


class StreamGraph:
    """One captured launch sequence on ``stream``, replayed as a HIP graph."""

    def __init__(self, record: Callable[[], None], stream: int) -> None:
        if not stream:
            raise ValueError("graph capture needs an explicit (non-null) HIP stream")
        self.stream = stream
        self._graph = self._exec = 0
        hip.capture_begin(stream)
        try:
            record()
        except BaseException:
            graph = hip.capture_end(stream)
            if graph:
                hip.library().hipGraphDestroy(graph)
            raise
        self._graph = hip.capture_end(stream)
        self._exec = hip.graph_instantiate(self._graph)

    @classmethod
    def profiled(cls, records: list[Callable[[], None]], stream: int, events: list[int]) -> "StreamGraph":
        """One capture of ``records`` with an event-record node before the first call, between
        consecutive calls and after the last (``events``, one more than calls): every replay
        writes each call's start and end."""
        if len(events) != len(records) + 1:
            raise ValueError("a profiled graph needs one event more than it has calls")

        def record() -> None:
            hip.capture_event(stream, events[0])
            for rec, event in zip(records, events[1:]):
                rec()
                hip.capture_event(stream, event)

        return cls(record, stream)

    def launch(self) -> None:
        """Enqueue one replay on the stream (asynchronous)."""
        if not self._exec:
            raise RuntimeError("graph is closed")
        hip.call("hipGraphLaunch", self._exec, self.stream)

    def __call__(self, wait: bool = False) -> float | None:
        """Replay once; with ``wait`` block until it finishes and return its GPU seconds."""
        if not wait:
            self.launch()
            return None
        start, stop = hip.event_create(), hip.event_create()
        try:
            hip.call("hipEventRecord", start, self.stream)
            self.launch()
            hip.call("hipEventRecord", stop, self.stream)
            hip.call("hipEventSynchronize", stop)
            return hip.elapsed_ms(start, stop) / 1e3
        finally:
            hip.call("hipEventDestroy", start)
            hip.call("hipEventDestroy", stop)

    def close(self) -> None:
        lib = hip.library()
        if self._exec:
            lib.hipGraphExecDestroy(self._exec)
        if self._graph:
            lib.hipGraphDestroy(self._graph)
        self._exec = self._graph = 0

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass


class MI355XGraph:
    """A fixed sequence of plugin program calls on one device, replayed as one HIP graph.

    ``calls`` holds ``(program, buffers, global_size, local_size, vals)`` tuples, the
    arguments of ``MI355XProgram.__call__``.
    """

    def __init__(self, calls: Sequence[tuple]) -> None:
        if not calls:
            raise ValueError("MI355X graphs need at least one program call")
        programs = [c[0] for c in calls]
        self.dev = programs[0].dev
        if any(p.dev is not self.dev for p in programs):
            raise ValueError("MI355X graphs require one device")
        self.lock = threading.RLock()
        self.calls = [self._normalise(c) for c in calls]
        self._graph: StreamGraph | None = None
        self._recorded: list[tuple] | None = None
        self._timing: profile.GraphTiming | None = None

    @staticmethod
    def _normalise(call: tuple) -> tuple:
        program, bufs, global_size, local_size, vals = call
        return program, tuple(bufs), tuple(global_size), tuple(local_size), tuple(vals)

    def _key(self, calls: list[tuple]) -> list[tuple]:
        # a graph captured with timestamp nodes is re-recorded when profiling is switched
        return [profile.enabled()] + [(id(p), tuple(id(b) for b in bufs), g, l, v) for p, bufs, g, l, v in calls]

    def _record(self, calls: list[tuple]) -> None:
        # validate every call exactly as an eager launch would, before capturing anything
        for program, bufs, global_size, local_size, vals in calls:
            program.validate(bufs, global_size, local_size, vals)

        if self._timing is not None:
            self._timing.close()
            self._timing = None
        with self.dev.lock:
            self.dev.select()
            timing = profile.GraphTiming(self.dev, [c[0].name for c in calls]) if profile.enabled() else None

            def record() -> None:
                for program, bufs, global_size, local_size, vals in calls:
                    program.enqueue(bufs, global_size, local_size, vals)

            if self._graph is not None:
                self._graph.close()
            if timing is None:
                self._graph = StreamGraph(record, self.dev.stream)
            else:
                one = [lambda c=c: c[0].enqueue(*c[1:]) for c in calls]
                self._graph = StreamGraph.profiled(one, self.dev.stream, timing.events)
            self._timing = timing
        self._recorded = self._key(calls)

    def __call__(self, updates: dict[int, tuple] | None = None, wait: bool = False) -> float | None:
        """Replay the sequence; ``updates`` maps a call index to new ``(buffers, global, local, vals)``.

        Returns GPU seconds when ``wait``.
        """
        with self.lock:
            calls = list(self.calls)
            for j, (bufs, global_size, local_size, vals) in (updates or {}).items():
                calls[j] = self._normalise((calls[j][0], bufs, global_size, local_size, vals))
            if self._graph is None or self._key(calls) != self._recorded:
                self._record(calls)
                self.calls = calls
            with self.dev.lock, self.dev.submitting():
                owners = tuple(b.owner for _, bufs, *_ in calls for b in bufs)
                if not wait and self._timing is None:
                    self._graph.launch()
                    self.dev.submitted(owners)
                    return None
                seconds = self._graph(wait=True)
                self.dev.submitted(owners)
                if self._timing is not None:  # this replay's signals, before another overwrites them
                    self._timing.publish()
                return seconds if wait else None

    def close(self) -> None:
        if self._graph is not None:
            self._graph.close()
            self._graph = None
        if self._timing is not None:
            self._timing.close()
            self._timing = None
