"""Per-kernel GPU timestamps published to a profiler.

The reference records a GPU timestamp pair around every eager launch and publishes it as a
``ProfileRangeEvent`` once the submission completes (alexandreteles/tinygrad-dx12
src/tinygrad_dx12/runtime/ops_dx12.py:120-147, :725-732); a recorded graph writes
``kernel_count + 1`` timestamps -- one before the first kernel and one after each -- and
publishes a ``ProfileGraphEvent`` of per-kernel entries over those signals
(runtime/graph/dx12.py:224, :249-253).  Both happen only under tinygrad's ``PROFILE``.

Here the timestamps are HIP events on the device stream.  A device records one reference
event when profiling starts (``DeviceClock``); every published time is microseconds after it,
as a ``decimal.Decimal`` like tinygrad's.  A graph captured under profiling gets an
event-record node before its first call, between calls and after the last
(``StreamGraph.profiled``; an event recorded during stream capture becomes no node on this
runtime, so the nodes are added to the capture graph), so every replay writes real per-call
times.  The events go to ``profile_events`` (tinygrad's
``Compiled.profile_events`` when tinygrad is importable, a module list otherwise), using
tinygrad's event classes when it is installed and field-for-field stand-ins when not.

Profiling is on when ``MI355X_PROFILE`` (or tinygrad's ``PROFILE``) is a non-zero integer, or
after ``set_enabled(True)``.
"""

from __future__ import annotations

import decimal
import os
import threading
from dataclasses import dataclass

from tinygrad_mi355x.runtime.support import hip

try:  # tinygrad's own profiler types and event list, when tinygrad is installed
    from tinygrad.device import Compiled, ProfileDeviceEvent  # type: ignore
    from tinygrad.helpers import ProfileGraphEntry, ProfileGraphEvent, ProfileRangeEvent  # type: ignore

    profile_events: list = Compiled.profile_events
except ImportError:  # stand-ins with tinygrad's fields
    @dataclass(frozen=True)
    class ProfileDeviceEvent:  # type: ignore[no-redef]
        device: str
        comp_tdiff: decimal.Decimal = decimal.Decimal(0)
        copy_tdiff: decimal.Decimal = decimal.Decimal(0)

    @dataclass(frozen=True)
    class ProfileRangeEvent:  # type: ignore[no-redef]
        device: str
        name: str
        st: decimal.Decimal
        en: decimal.Decimal | None
        is_copy: bool = False

    @dataclass(frozen=True)
    class ProfileGraphEntry:  # type: ignore[no-redef]
        device: str
        name: str
        st_id: int
        en_id: int
        is_copy: bool

    @dataclass(frozen=True)
    class ProfileGraphEvent:  # type: ignore[no-redef]
        ents: list
        deps: list
        sigs: list

    profile_events = []

def _env_flag() -> bool:
    for name in ("MI355X_PROFILE", "PROFILE"):
        value = os.environ.get(name, "").strip()
        if value:
            try:
                return int(value) != 0
            except ValueError:
                return False
    return False


_enabled = _env_flag()


def enabled() -> bool:
    return _enabled


def set_enabled(on: bool) -> None:
    """Turn timestamp publishing on or off for launches made from now on."""
    global _enabled
    _enabled = bool(on)


def _us(ms: float) -> decimal.Decimal:
    return decimal.Decimal(repr(ms)) * 1000


class DeviceClock:
    """The reference event of one device: published times are microseconds after it."""

    def __init__(self, dev) -> None:
        self.device = dev.device
        self.ref = hip.event_create()
        hip.call("hipEventRecord", self.ref, dev.stream)
        hip.call("hipEventSynchronize", self.ref)
        profile_events.append(ProfileDeviceEvent(dev.device))

    def since(self, event: int) -> decimal.Decimal:
        return _us(hip.elapsed_ms(self.ref, event))


_clock_lock = threading.Lock()


def clock(dev) -> DeviceClock:
    """The device's clock, created on first use (the caller holds the device lock)."""
    with _clock_lock:
        c = getattr(dev, "_profile_clock", None)
        if c is None:
            c = DeviceClock(dev)
            dev._profile_clock = c
        return c


class RangeTiming:
    """A timestamp pair around one eager launch; ``publish`` runs after it completed."""

    def __init__(self, dev, name: str) -> None:
        self.clock, self.name, self.device = clock(dev), name, dev.device
        self.start, self.stop = hip.event_create(), hip.event_create()
        hip.call("hipEventRecord", self.start, dev.stream)

    def end(self, dev) -> None:
        hip.call("hipEventRecord", self.stop, dev.stream)

    def publish(self) -> None:
        try:
            st = self.clock.since(self.start)
            profile_events.append(ProfileRangeEvent(self.device, self.name, st,
                                                    st + _us(hip.elapsed_ms(self.start, self.stop))))
        finally:
            hip.call("hipEventDestroy", self.start)
            hip.call("hipEventDestroy", self.stop)


class GraphTiming:
    """``count + 1`` events for a graph of ``count`` calls (event i is recorded before call i,
    the last after the last call); ``publish`` reads one replay's signals."""

    def __init__(self, dev, names: list[str]) -> None:
        self.clock, self.device, self.names = clock(dev), dev.device, list(names)
        self.events = [hip.event_create() for _ in range(len(names) + 1)]

    def signals(self) -> list[decimal.Decimal]:
        first = self.clock.since(self.events[0])
        return [first] + [first + _us(hip.elapsed_ms(self.events[0], e)) for e in self.events[1:]]

    def publish(self) -> ProfileGraphEvent:
        sigs = self.signals()
        ents = [ProfileGraphEntry(self.device, name, i, i + 1, False) for i, name in enumerate(self.names)]
        deps = [[i - 1] if i else [] for i in range(len(self.names))]  # a stream runs them in order
        event = ProfileGraphEvent(ents, deps, sigs)
        profile_events.append(event)
        return event

    def close(self) -> None:
        for e in self.events:
            hip.call("hipEventDestroy", e)
        self.events = []


def kernel_seconds(event) -> list[float]:
    """Per-kernel GPU seconds of a published ``ProfileGraphEvent``."""
    return [float(event.sigs[e.en_id] - event.sigs[e.st_id]) / 1e6 for e in event.ents]
