"""Device buffers and stream-ordered timing through the library's own C ABI
(spinn_hip_malloc / memcpy / events), for callers that do not use torch."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import native as N


class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.L = N.lib()
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        N.check(self.L.spinn_hip_malloc(C.byref(p), max(self.nbytes, 4)), "spinn_hip_malloc")
        self.ptr = p

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        N.check(self.L.spinn_hip_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, None), "h2d")
        N.check(self.L.spinn_hip_stream_sync(None), "sync")

    def download(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        N.check(self.L.spinn_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, None), "d2h")
        N.check(self.L.spinn_hip_stream_sync(None), "sync")
        return out

    def free(self) -> None:
        if self.ptr:
            self.L.spinn_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def time_launches(fn, reps: int, warmup: int = 3, stream=None) -> float:
    """Mean milliseconds per call of `fn` (which enqueues work on `stream`),
    from two HIP events recorded around `reps` back-to-back calls."""
    L = N.lib()
    for _ in range(warmup):
        fn()
    e0, e1 = C.c_void_p(), C.c_void_p()
    N.check(L.spinn_hip_event_create(C.byref(e0)), "event")
    N.check(L.spinn_hip_event_create(C.byref(e1)), "event")
    try:
        N.check(L.spinn_hip_stream_sync(stream), "sync")
        N.check(L.spinn_hip_event_record(e0, stream), "record")
        for _ in range(reps):
            fn()
        N.check(L.spinn_hip_event_record(e1, stream), "record")
        ms = C.c_float()
        N.check(L.spinn_hip_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
        return ms.value / reps
    finally:
        L.spinn_hip_event_destroy(e0)
        L.spinn_hip_event_destroy(e1)


def time_cold(fn, flush, reps: int) -> float:
    """Mean milliseconds of one call of `fn` right after `flush` (work that evicts
    the caches, e.g. a copy larger than the Infinity Cache): events bracket `fn`
    alone, `reps` times, on the null stream."""
    L = N.lib()
    e0, e1 = C.c_void_p(), C.c_void_p()
    N.check(L.spinn_hip_event_create(C.byref(e0)), "event")
    N.check(L.spinn_hip_event_create(C.byref(e1)), "event")
    total = 0.0
    try:
        for _ in range(reps):
            flush()
            N.check(L.spinn_hip_event_record(e0, None), "record")
            N.check(fn(), "timed call")
            N.check(L.spinn_hip_event_record(e1, None), "record")
            N.check(L.spinn_hip_stream_sync(None), "sync")
            ms = C.c_float()
            N.check(L.spinn_hip_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
            total += ms.value
    finally:
        L.spinn_hip_event_destroy(e0)
        L.spinn_hip_event_destroy(e1)
    return total / reps


def time_graph(fn, reps: int, replays: int = 5) -> float:
    """Mean milliseconds per call of `fn(stream)` measured GPU-side: `reps` calls
    are captured into one HIP graph on a stream of their own and the graph is
    replayed `replays` times between two HIP events on that stream, so the
    figure carries no host launch gap between the calls (which dominates
    back-to-back launches of kernels of a few microseconds)."""
    L = N.lib()
    st = C.c_void_p()
    N.check(L.spinn_hip_stream_create(C.byref(st)), "stream")
    g = C.c_void_p()
    e0, e1 = C.c_void_p(), C.c_void_p()
    N.check(L.spinn_hip_event_create(C.byref(e0)), "event")
    N.check(L.spinn_hip_event_create(C.byref(e1)), "event")
    try:
        N.check(fn(st), "warm-up call")
        N.check(L.spinn_hip_stream_sync(st), "sync")
        N.check(L.spinn_hip_graph_capture_begin(st), "capture")
        rcs = [fn(st) for _ in range(reps)]
        N.check(L.spinn_hip_graph_capture_end(st, C.byref(g)), "capture end")
        for rc in rcs:
            N.check(rc, "captured call")
        N.check(L.spinn_hip_graph_launch(g, st), "replay")
        N.check(L.spinn_hip_event_record(e0, st), "record")
        for _ in range(replays):
            N.check(L.spinn_hip_graph_launch(g, st), "replay")
        N.check(L.spinn_hip_event_record(e1, st), "record")
        N.check(L.spinn_hip_stream_sync(st), "sync")
        ms = C.c_float()
        N.check(L.spinn_hip_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
        return ms.value / (reps * replays)
    finally:
        if g:
            L.spinn_hip_graph_destroy(g)
        L.spinn_hip_event_destroy(e0)
        L.spinn_hip_event_destroy(e1)
        L.spinn_hip_stream_destroy(st)
