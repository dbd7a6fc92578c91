"""Runtime tier: device, buffers, streams, events.

Python face of the ironmill-metal-sys counterpart in the C ABI
(ironmill-metal-sys/src/{device,buffer,command}.rs).  Objects own their
native handles and release them when closed or garbage-collected.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import DeviceInfo, check, lib


class Device:
    """MetalDevice counterpart (device.rs:63-513) for one HIP device."""

    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        check(lib.imh_device_open(ordinal, C.byref(h)))
        self._h = h

    @staticmethod
    def count() -> int:
        n = C.c_int(0)
        rc = lib.imh_device_count(C.byref(n))
        return n.value if rc == 0 else 0

    @property
    def handle(self):
        return self._h

    def info(self) -> dict:
        inf = DeviceInfo()
        check(lib.imh_device_get_info(self._h, C.byref(inf)))
        return {
            "ordinal": inf.ordinal,
            "compute_units": inf.compute_units,
            "wavefront_size": inf.wavefront_size,
            "clock_khz": inf.clock_khz,
            "total_global_mem": inf.total_global_mem,
            "lds_per_block": inf.lds_per_block,
            "arch": inf.arch.decode(),
        }

    def buffer(self, nbytes: int) -> "Buffer":
        return Buffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> "Buffer":
        """create_buffer_with_data: a device copy of a host array (dtype/shape kept)."""
        arr = np.ascontiguousarray(arr)
        buf = Buffer(self, max(arr.nbytes, 1))
        if arr.nbytes:
            buf.write(arr)
        buf.dtype, buf.shape = arr.dtype, arr.shape
        return buf

    def empty(self, shape, dtype) -> "Buffer":
        dtype = np.dtype(dtype)
        n = int(np.prod(shape)) * dtype.itemsize
        buf = Buffer(self, max(n, 1))
        buf.dtype, buf.shape = dtype, tuple(shape)
        return buf

    def stream(self) -> "Stream":
        return Stream(self)

    def event(self) -> "Event":
        return Event(self)

    def close(self):
        if getattr(self, "_h", None):
            lib.imh_device_free(self._h)
            self._h = None

    def __del__(self):
        self.close()


class Buffer:
    """MetalBuffer counterpart (buffer.rs:42-168): bounds-checked device memory."""

    def __init__(self, dev: Device, nbytes: int):
        h = C.c_void_p()
        check(lib.imh_buffer_alloc(dev.handle, nbytes, C.byref(h)))
        self._h = h
        self._dev = dev  # keep the device alive
        self.dtype = np.dtype(np.uint8)
        self.shape = (nbytes,)

    @property
    def ptr(self) -> int:
        return lib.imh_buffer_device_ptr(self._h)

    @property
    def nbytes(self) -> int:
        return lib.imh_buffer_length(self._h)

    def write(self, arr: np.ndarray, offset: int = 0):
        arr = np.ascontiguousarray(arr)
        check(lib.imh_buffer_write(self._h, offset, arr.ctypes.data_as(C.c_void_p), arr.nbytes))

    def read(self, dtype=None, shape=None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype or self.dtype)
        shape = tuple(shape) if shape is not None else self.shape
        out = np.empty(shape, dtype)
        check(lib.imh_buffer_read(self._h, offset, out.ctypes.data_as(C.c_void_p), out.nbytes))
        return out

    def close(self):
        if getattr(self, "_h", None):
            lib.imh_buffer_free(self._h)
            self._h = None

    def __del__(self):
        self.close()


class Stream:
    """CommandQueue counterpart (command.rs:16-130): an in-order HIP stream."""

    def __init__(self, dev: Device):
        h = C.c_void_p()
        check(lib.imh_stream_create(dev.handle, C.byref(h)))
        self._h = h
        self._dev = dev

    @property
    def handle(self):
        return self._h

    def sync(self):
        check(lib.imh_stream_sync(self._h))

    def zero(self, buf: Buffer):
        check(lib.imh_fill_zero(self._h, buf.ptr, buf.nbytes))

    def capture(self, fn) -> "Graph":
        """Record the ops fn() encodes on this stream into a replayable graph."""
        check(lib.imh_stream_begin_capture(self._h))
        try:
            fn()
        except BaseException:
            g = C.c_void_p()
            lib.imh_stream_end_capture(self._h, C.byref(g))
            if g:
                lib.imh_graph_free(g)
            raise
        g = C.c_void_p()
        check(lib.imh_stream_end_capture(self._h, C.byref(g)))
        return Graph(g, self)

    def close(self):
        if getattr(self, "_h", None):
            lib.imh_stream_free(self._h)
            self._h = None

    def __del__(self):
        self.close()


class Graph:
    """A captured op sequence (imh_graph): replay with launch()."""

    def __init__(self, handle, stream: Stream):
        self._h = handle
        self._stream = stream

    def launch(self, stream: Stream | None = None):
        check(lib.imh_graph_launch(self._h, (stream or self._stream).handle))

    def close(self):
        if getattr(self, "_h", None):
            lib.imh_graph_free(self._h)
            self._h = None

    def __del__(self):
        self.close()


class Event:
    """gpu_start_time / gpu_end_time counterpart (command.rs:470-489)."""

    def __init__(self, dev: Device):
        h = C.c_void_p()
        check(lib.imh_event_create(dev.handle, C.byref(h)))
        self._h = h
        self._dev = dev

    def record(self, stream: Stream):
        check(lib.imh_event_record(self._h, stream.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib.imh_event_elapsed_ms(self._h, end._h, C.byref(ms)))
        return ms.value

    def close(self):
        if getattr(self, "_h", None):
            lib.imh_event_free(self._h)
            self._h = None

    def __del__(self):
        self.close()
