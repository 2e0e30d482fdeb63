"""torch.profiler for the 'hip' device (src/profiler/index.ts).

The reference's record_function measures host time up to the WebGPU
submission (index.ts:145-166).  Here each block is also a named range on
the ROCm tracer's marker timeline (roctx, through tjh_range_push/pop:
`rocprofv3 --marker-trace` shows it around the kernels launched inside)
and carries a pair of HIP events on the library stream, so an event
records both its host time and its device time.  Device times are read
when the profiler stops (stop synchronises, like the reference's
syncDevice in Profiler.stop, index.ts:111-115), not inside the block.
"""
import ctypes
import time
from enum import Enum

from . import _lib as L


class ProfilerActivity(str, Enum):
    """index.ts:4-8 (CUDA and WEBGPU are aliases of the device timeline)."""
    CPU = "cpu"
    CUDA = "cuda"
    WEBGPU = "webgpu"
    HIP = "hip"


class ProfilerEvent(dict):
    """One recorded block (index.ts:17-25): name, activity, start, end and
    duration (host ms), device_duration (ms between the block's stream
    events), memory_usage (change of the allocator's active bytes)."""

    __getattr__ = dict.get


def _active_bytes():
    s = L.MemStats()
    L.check(L.lib().tjh_memory_stats(ctypes.byref(s)), "memory_stats")
    return int(s.active_bytes)


class KinetoStep:
    """Events grouped by name (index.ts:30-72)."""

    def __init__(self, events):
        self.events = list(events)

    def key_averages(self, group_by_input_shape=False):
        return self

    def stats(self):
        out = {}
        for e in self.events:
            st = out.setdefault(e["name"], {"count": 0, "total_duration": 0.0,
                                            "total_device_duration": 0.0, "total_memory": 0})
            st["count"] += 1
            st["total_duration"] += e.get("duration") or 0.0
            st["total_device_duration"] += e.get("device_duration") or 0.0
            st["total_memory"] += e.get("memory_usage") or 0
        return out

    def table(self, sort_by="duration", row_limit=50):
        key = "total_device_duration" if sort_by in ("device_duration", "cuda_time_total",
                                                      "self_cuda_time_total") \
            else "total_duration"
        rows = sorted(self.stats().items(), key=lambda kv: -kv[1][key])[:row_limit]
        lines = ["", "-" * 78,
                 "%-30s | %8s | %12s | %12s | %10s" % ("Name", "Count", "Host Time",
                                                       "Device Time", "Mem"),
                 "-" * 78]
        for name, d in rows:
            lines.append("%-30s | %8d | %9.3f ms | %9.3f ms | %7.0f KB" % (
                name[:30], d["count"], d["total_duration"], d["total_device_duration"],
                d["total_memory"] / 1024.0))
        lines.append("-" * 78)
        return "\n".join(lines)


_active = [None]


class Profiler:
    """index.ts:80-131: collects record_function events between start() and
    stop()."""

    def __init__(self, activities=None, record_shapes=False, profile_memory=False,
                 with_stack=False):
        self.options = {"activities": activities or [ProfilerActivity.CPU, ProfilerActivity.HIP],
                        "record_shapes": record_shapes, "profile_memory": profile_memory,
                        "with_stack": with_stack}
        self.events = []
        self.active = False
        self._pending = []  # (event, timer id) awaiting device times

    def start(self):
        self.events = []
        self._pending = []
        self.active = True
        _active[0] = self

    def stop(self):
        L.check(L.lib().tjh_synchronize(), "synchronize")
        for ev, tid in self._pending:
            ms = ctypes.c_double(0.0)
            L.check(L.lib().tjh_timer_read(tid, ctypes.byref(ms)), "timer_read")
            ev["device_duration"] = ms.value
        self._pending = []
        self.active = False
        if _active[0] is self:
            _active[0] = None

    def _record_event(self, event, timer=None):
        if self.active:
            self.events.append(event)
            if timer is not None:
                self._pending.append((event, timer))

    def get_events(self):
        return self.events

    def key_averages(self):
        return KinetoStep(self.events)

    def __enter__(self):
        self.start()
        return self

    def __exit__(self, *exc):
        self.stop()
        return False


def profile(options=None, fn=None, **kwargs):
    """profile(options, fn) as in index.ts:136-150 (runs fn(profiler) and
    returns the stopped profiler), or a context manager:
    `with profile() as p: ...`."""
    if callable(options) and fn is None:
        options, fn = None, options
    p = Profiler(**(options or {}), **kwargs)
    if fn is None:
        return p
    p.start()
    try:
        fn(p)
    finally:
        p.stop()
    return p


class record_function:
    """record_function(name, fn) (index.ts:155-182) returns fn()'s result
    with the block recorded; `with record_function(name):` and the
    decorator form work too.  The block is always a roctx range (visible to
    rocprofv3 --marker-trace); it becomes an event only while a profiler is
    active."""

    def __new__(cls, name, fn=None):
        self = super().__new__(cls)
        self.name = str(name)
        if fn is not None:
            with self:
                return fn()
        return self

    def __enter__(self):
        lib = L.lib()
        L.check(lib.tjh_range_push(self.name.encode()), "range_push")
        self._prof = _active[0] if _active[0] is not None and _active[0].active else None
        self._timer = None
        if self._prof is not None:
            tid = ctypes.c_int(0)
            L.check(lib.tjh_timer_start(ctypes.byref(tid)), "timer_start")
            self._timer = tid.value
            self._mem0 = _active_bytes()
        self._t0 = time.perf_counter()
        return self

    def __exit__(self, *exc):
        t1 = time.perf_counter()
        lib = L.lib()
        if self._timer is not None:
            L.check(lib.tjh_timer_end(self._timer), "timer_end")
            ev = ProfilerEvent(name=self.name, activity=ProfilerActivity.HIP.value,
                               start=self._t0 * 1e3, end=t1 * 1e3,
                               duration=(t1 - self._t0) * 1e3,
                               memory_usage=_active_bytes() - self._mem0)
            self._prof._record_event(ev, self._timer)
        L.check(lib.tjh_range_pop(), "range_pop")
        return False

    def __call__(self, fn):
        name = self.name

        def wrapped(*a, **k):
            with record_function(name):
                return fn(*a, **k)
        wrapped.__name__ = getattr(fn, "__name__", name)
        return wrapped


def record_function_async(name, fn):
    """index.ts:187-210: the block, then a device synchronisation."""
    with record_function(name):
        out = fn()
    L.check(L.lib().tjh_synchronize(), "synchronize")
    return out


def mark(name):
    """A point marker on the roctx timeline."""
    L.check(L.lib().tjh_mark(str(name).encode()), "mark")
