"""Device memory, streams and events over the library's own HIP plumbing (``brasa_hip_rt.h``).

They stand in for the reference's ``brasa_metal`` ``Buffer`` / ``Command`` / GPU timing
(crates/metal/src/runtime.rs:134-425). Using the library's HIP runtime for these keeps exactly
one HIP runtime in the process.
"""
from __future__ import annotations

import contextlib
import ctypes

import numpy as np

from ._lib import VP, check, lib


def device_count() -> int:
    n = ctypes.c_int(0)
    st = lib().brasa_rt_device_count(ctypes.byref(n))
    return n.value if st == 0 else 0


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    check(lib().brasa_rt_device_name(buf, 256))
    return buf.value.decode()


def mem_info() -> tuple[int, int]:
    """(free, total) bytes of the current device."""
    f, t = ctypes.c_size_t(0), ctypes.c_size_t(0)
    check(lib().brasa_rt_mem_info(ctypes.byref(f), ctypes.byref(t)))
    return int(f.value), int(t.value)


def synchronize() -> None:
    check(lib().brasa_rt_device_synchronize())


class DeviceBuffer:
    """A hipMalloc'ed byte buffer; ``ptr`` is the device address as an int."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = VP()
        check(lib().brasa_rt_malloc(ctypes.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().brasa_rt_memcpy_htod(self.ptr + offset, a.ctypes.data, a.nbytes))

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().brasa_rt_memcpy_dtoh(out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def fill(self, value: int, stream: "Stream | None" = None) -> None:
        check(lib().brasa_rt_fill_u8(self.ptr, value, self.nbytes, stream.handle if stream else None))

    def free(self) -> None:
        if self.ptr:
            check(lib().brasa_rt_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr:
                lib().brasa_rt_free(self.ptr)
                self.ptr = 0
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = VP()
        check(lib().brasa_rt_stream_create(ctypes.byref(s)))
        self.handle = s.value

    def synchronize(self) -> None:
        check(lib().brasa_rt_stream_synchronize(self.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().brasa_rt_stream_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Graph:
    """A HIP graph captured from the work one block enqueues on a stream:

        with Graph.capture(stream) as g:
            kernels.decode_attention_lanes(..., stream=stream)
        g.launch(stream)   # replays the captured launches
    """

    def __init__(self):
        self.handle = None

    @classmethod
    @contextlib.contextmanager
    def capture(cls, stream: Stream):
        g = cls()
        check(lib().brasa_rt_stream_begin_capture(stream.handle))
        try:
            yield g
        finally:
            h = VP()
            check(lib().brasa_rt_stream_end_capture(stream.handle, ctypes.byref(h)))
            g.handle = h.value

    def launch(self, stream: Stream) -> None:
        check(lib().brasa_rt_graph_launch(self.handle, stream.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().brasa_rt_graph_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Event:
    def __init__(self):
        e = VP()
        check(lib().brasa_rt_event_create(ctypes.byref(e)))
        self.handle = e.value

    def record(self, stream: Stream | None = None) -> None:
        check(lib().brasa_rt_event_record(self.handle, stream.handle if stream else None))

    def synchronize(self) -> None:
        check(lib().brasa_rt_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0)
        check(lib().brasa_rt_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle))
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                lib().brasa_rt_event_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


def fill_normal(buf: DeviceBuffer, n: int, seed: int, scale: float = 1.0,
                stream: Stream | None = None, offset: int = 0) -> None:
    """Synthetic N(0, scale^2) f32 values generated on the device (benchmarks only)."""
    assert offset + 4 * n <= buf.nbytes
    check(lib().brasa_rt_fill_normal_f32(buf.ptr + offset, n, seed, scale,
                                         stream.handle if stream else None))
