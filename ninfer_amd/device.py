"""Device memory, streams, events and graphs through the library's runtime helpers.

Plumbing for harnesses (tests, benchmark): no other GPU framework is involved, so the process
uses exactly the HIP runtime the library was built against.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _capi
from ._capi import Tensor, check, lib

_NP_DTYPE = {
    _capi.BF16: np.uint16,
    _capi.FP16: np.uint16,
    _capi.FP32: np.float32,
    _capi.I8: np.int8,
    _capi.I32: np.int32,
    _capi.I64: np.int64,
}


def device_count() -> int:
    n = C.c_int32(0)
    check(lib().nmi_rt_device_count(C.byref(n)))
    return int(n.value)


def device_name() -> str:
    buf = C.create_string_buffer(256)
    check(lib().nmi_rt_device_name(buf, 256))
    return buf.value.decode()


class DeviceBuffer:
    """Owning device allocation (hipMalloc'd, 256-byte aligned)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().nmi_rt_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = int(p.value)

    def free(self) -> None:
        if self.ptr:
            check(lib().nmi_rt_free(C.c_void_p(self.ptr)))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes, "upload out of range"
        check(lib().nmi_rt_memcpy_htod(C.c_void_p(self.ptr + offset), a.ctypes.data_as(C.c_void_p), a.nbytes))

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes, "download out of range"
        check(lib().nmi_rt_memcpy_dtoh(out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr + offset), out.nbytes))
        return out

    def fill(self, value: int = 0, stream: "Stream | None" = None) -> None:
        check(lib().nmi_rt_fill_u8(C.c_void_p(self.ptr), value, self.nbytes, stream.handle if stream else None))


class DeviceArray:
    """A device buffer with a dtype and a reference-order shape (ne[0] fastest)."""

    def __init__(self, dtype: int, shape, buf: DeviceBuffer | None = None, offset: int = 0):
        self.dtype = dtype
        self.shape = tuple(int(s) for s in shape)
        self.count = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.count * _capi.DTYPE_SIZE[dtype]
        self.buf = buf if buf is not None else DeviceBuffer(self.nbytes)
        self.offset = offset

    @property
    def ptr(self) -> int:
        return self.buf.ptr + self.offset

    @classmethod
    def from_numpy(cls, dtype: int, arr: np.ndarray, shape=None) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        if shape is None:
            shape = tuple(reversed(arr.shape)) if arr.ndim else (1,)
        d = cls(dtype, shape)
        d.upload(arr)
        return d

    def upload(self, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr).view(_NP_DTYPE[self.dtype]).reshape(-1)
        assert a.size == self.count, f"size mismatch {a.size} vs {self.count}"
        self.buf.upload(a, self.offset)

    def numpy(self) -> np.ndarray:
        return self.buf.download(_NP_DTYPE[self.dtype], self.count, self.offset)

    def tensor(self) -> Tensor:
        return Tensor.make(self.ptr, self.dtype, self.shape)

    def zero(self, stream: "Stream | None" = None) -> None:
        check(lib().nmi_rt_fill_u8(C.c_void_p(self.ptr), 0, self.nbytes, stream.handle if stream else None))


class Stream:
    def __init__(self):
        h = C.c_void_p()
        check(lib().nmi_rt_stream_create(C.byref(h)))
        self.handle = h.value

    def synchronize(self) -> None:
        check(lib().nmi_rt_stream_synchronize(self.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().nmi_rt_stream_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Event:
    def __init__(self):
        h = C.c_void_p()
        check(lib().nmi_rt_event_create(C.byref(h)))
        self.handle = h.value

    def record(self, stream: Stream | None) -> None:
        check(lib().nmi_rt_event_record(self.handle, stream.handle if stream else None))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        check(lib().nmi_rt_event_elapsed_ms(C.byref(ms), self.handle, end.handle))
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                lib().nmi_rt_event_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Graph:
    """Capture a sequence of calls on `stream` into a replayable HIP graph."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self.handle = None

    def __enter__(self):
        check(lib().nmi_rt_capture_begin(self.stream.handle))
        return self

    def __exit__(self, exc_type, exc, tb):
        h = C.c_void_p()
        check(lib().nmi_rt_capture_end(self.stream.handle, C.byref(h)))
        self.handle = h.value
        return False

    def launch(self) -> None:
        check(lib().nmi_rt_graph_launch(self.handle, self.stream.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().nmi_rt_graph_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


def synchronize() -> None:
    check(lib().nmi_rt_device_synchronize())


def copy_array(dst: "DeviceArray", src: "DeviceArray", stream: Stream | None = None) -> None:
    """Stream-ordered copy of src's bytes into dst (same byte size; either may live in an arena)."""
    assert dst.nbytes == src.nbytes
    check(lib().nmi_rt_memcpy_dtod(C.c_void_p(dst.ptr), C.c_void_p(src.ptr), dst.nbytes,
                                   stream.handle if stream else None))


def next_row_i32(table: "DeviceArray", counter: "DeviceArray", dst: "DeviceArray", stream: Stream | None = None) -> None:
    """dst <- row (counter mod rows) of the int32 table (shape (cols, rows), rows contiguous), then
    counter + 1 (on the device)."""
    cols, rows = table.shape[0], table.shape[1]
    check(lib().nmi_rt_next_row_i32(C.c_void_p(table.ptr), rows, cols, C.c_void_p(counter.ptr), C.c_void_p(dst.ptr),
                                    stream.handle if stream else None))


READ_VECTOR, READ_LDS_DMA = 0, 1


def stream_copy(dst_ptr: int, src_ptr: int, nbytes: int, stream: Stream | None = None) -> None:
    """Copy-ceiling control: one launch of 16-byte loads and stores over `nbytes`."""
    check(lib().nmi_rt_stream_copy(C.c_void_p(dst_ptr), C.c_void_p(src_ptr), nbytes,
                                   stream.handle if stream else None))


def read_ceiling(src_ptr: int, nbytes: int, form: int, sink: DeviceBuffer, stream: Stream | None = None) -> None:
    """Read-ceiling control: one launch that reads `nbytes` (READ_VECTOR or READ_LDS_DMA)."""
    check(lib().nmi_rt_read_ceiling(C.c_void_p(src_ptr), nbytes, form, C.c_void_p(sink.ptr),
                                    stream.handle if stream else None))


def memcpy_dtod(dst: DeviceBuffer, src: DeviceBuffer, nbytes: int, stream: Stream | None = None) -> None:
    """Stream-ordered device-to-device copy of `nbytes` (hipMemcpyAsync)."""
    assert nbytes <= dst.nbytes and nbytes <= src.nbytes
    check(lib().nmi_rt_memcpy_dtod(C.c_void_p(dst.ptr), C.c_void_p(src.ptr), nbytes,
                                   stream.handle if stream else None))
