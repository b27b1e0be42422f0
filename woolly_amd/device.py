"""Device memory, streams and events through the C ABI (no PyTorch)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

_initialized: set[int] = set()


def init(device: int = 0) -> None:
    """Selects `device` for this thread and checks that it is a gfx950."""
    lib = _lib.load()
    _lib.check(lib.wh_init(device))
    _initialized.add(device)


def device_count() -> int:
    n = C.c_int(0)
    st = _lib.load().wh_device_count(C.byref(n))
    return n.value if st == _lib.WH_OK else 0


def device_name() -> str:
    buf = C.create_string_buffer(256)
    _lib.check(_lib.load().wh_device_name(buf, 256))
    return buf.value.decode()


def synchronize() -> None:
    _lib.check(_lib.load().wh_device_synchronize())


class DeviceBuffer:
    """An owned device allocation of `nbytes` (wh_malloc / wh_free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _lib.check(_lib.load().wh_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, arr: np.ndarray, stream: "Stream | None" = None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr, stream)
        return buf

    def upload(self, arr: np.ndarray, stream: "Stream | None" = None, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload exceeds the buffer")
        s = stream.handle if stream else None
        _lib.check(_lib.load().wh_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes, s))
        if stream is None:
            synchronize()

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            _lib.check(_lib.load().wh_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes,
                                                 None))
            synchronize()
        return out

    def fill(self, value: int = 0, stream: "Stream | None" = None) -> None:
        s = stream.handle if stream else None
        _lib.check(_lib.load().wh_fill_bytes(self.ptr, value, self.nbytes, s))
        if stream is None:
            synchronize()  # the library's streams do not wait for the null stream

    def free(self) -> None:
        if self.ptr:
            _lib.check(_lib.load().wh_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr:
                _lib.load().wh_free(self.ptr)
                self.ptr = 0
        except Exception:
            pass


class Stream:
    def __init__(self):
        h = C.c_void_p()
        _lib.check(_lib.load().wh_stream_create(C.byref(h)))
        self.handle = h.value

    def synchronize(self) -> None:
        _lib.check(_lib.load().wh_stream_synchronize(self.handle))

    def destroy(self) -> None:
        if self.handle:
            _lib.check(_lib.load().wh_stream_destroy(self.handle))
            self.handle = None


class Event:
    def __init__(self):
        h = C.c_void_p()
        _lib.check(_lib.load().wh_event_create(C.byref(h)))
        self.handle = h.value

    def record(self, stream: Stream | None = None) -> None:
        _lib.check(_lib.load().wh_event_record(self.handle, stream.handle if stream else None))

    def synchronize(self) -> None:
        _lib.check(_lib.load().wh_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _lib.check(_lib.load().wh_event_elapsed_ms(C.byref(ms), self.handle, end.handle))
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            _lib.check(_lib.load().wh_event_destroy(self.handle))
            self.handle = None


class Graph:
    """A captured sequence of stream-ordered calls, replayed with one launch.

        with Graph.capture(stream) as g:
            ops.quantized_matvec(..., stream=stream)
        g.launch(stream)
    """

    def __init__(self):
        self.handle = None

    @classmethod
    def capture(cls, stream: Stream) -> "_Capture":
        return _Capture(cls(), stream)

    def launch(self, stream: Stream) -> None:
        _lib.check(_lib.load().wh_graph_launch(self.handle, stream.handle))

    def destroy(self) -> None:
        if self.handle:
            _lib.check(_lib.load().wh_graph_destroy(self.handle))
            self.handle = None


class _Capture:
    def __init__(self, graph: Graph, stream: Stream):
        self.graph, self.stream = graph, stream

    def __enter__(self) -> Graph:
        _lib.check(_lib.load().wh_graph_begin_capture(self.stream.handle))
        return self.graph

    def __exit__(self, exc_type, exc, tb):
        h = C.c_void_p()
        st = _lib.load().wh_graph_end_capture(self.stream.handle, C.byref(h))
        if exc_type is None:
            _lib.check(st)
            self.graph.handle = h.value
        return False
