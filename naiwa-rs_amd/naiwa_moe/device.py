"""Device memory, pinned host memory, streams and events through the C ABI.

The library brings its own plumbing so the product path needs no framework:
a DeviceBuffer is a hipMalloc'd range owned by Python, a Stream/Event wraps
the hipStream_t/hipEvent_t handles the kernels take as int64.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib


def device_count() -> int:
    n = C.c_int(0)
    rc = lib().naiwa_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def device_info(dev: int = 0) -> dict:
    cu, khz, mem = C.c_int(0), C.c_int(0), C.c_int64(0)
    name = C.create_string_buffer(64)
    check(lib().naiwa_device_info(dev, C.byref(cu), C.byref(khz), C.byref(mem), name, 64), "device_info")
    return {"cu_count": cu.value, "wall_clock_khz": khz.value, "hbm_bytes": mem.value,
            "arch": name.value.decode()}


def mem_info() -> tuple[int, int]:
    """(free, total) bytes of the current device."""
    f, t = C.c_uint64(0), C.c_uint64(0)
    check(lib().naiwa_mem_info(C.byref(f), C.byref(t)), "mem_info")
    return f.value, t.value


def synchronize() -> None:
    check(lib().naiwa_device_sync(), "device sync")


class DeviceBuffer:
    """A device allocation of `nbytes` (256-B aligned)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().naiwa_malloc(C.byref(p), max(self.nbytes, 1)), f"malloc({nbytes})")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray, stream: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a, stream)
        return buf

    def upload(self, a: np.ndarray, stream: int = 0, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().naiwa_memcpy_h2d(self.ptr + offset, a.ctypes.data, a.nbytes, stream), "h2d")
        if stream == 0:
            check(lib().naiwa_stream_sync(0), "sync")

    def download(self, dtype, count: int | None = None, offset: int = 0, stream: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        check(lib().naiwa_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes, stream), "d2h")
        check(lib().naiwa_stream_sync(stream), "sync")
        return out

    def zero(self, stream: int = 0) -> None:
        check(lib().naiwa_memset(self.ptr, 0, self.nbytes, stream), "memset")

    def free(self) -> None:
        if self.ptr:
            lib().naiwa_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PinnedBuffer:
    """Pinned, portable host memory (hipHostMalloc) viewed as a numpy array."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().naiwa_host_alloc(C.byref(p), max(self.nbytes, 1)), f"host_alloc({nbytes})")
        self.ptr = p.value

    def view(self, dtype=np.uint8) -> np.ndarray:
        dtype = np.dtype(dtype)
        arr = (C.c_uint8 * self.nbytes).from_address(self.ptr)
        return np.frombuffer(arr, dtype=np.uint8).view(dtype)

    def free(self) -> None:
        if self.ptr:
            lib().naiwa_host_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        h = C.c_int64(0)
        check(lib().naiwa_stream_create(C.byref(h)), "stream_create")
        self.handle = h.value

    def sync(self) -> None:
        check(lib().naiwa_stream_sync(self.handle), "stream_sync")

    def wait(self, event: "Event") -> None:
        check(lib().naiwa_stream_wait_event(self.handle, event.handle), "stream_wait_event")

    def destroy(self) -> None:
        if self.handle:
            lib().naiwa_stream_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self, timing: bool = True):
        h = C.c_int64(0)
        check(lib().naiwa_event_create(C.byref(h), 1 if timing else 0), "event_create")
        self.handle = h.value

    def record(self, stream: int = 0) -> None:
        check(lib().naiwa_event_record(self.handle, stream), "event_record")

    def sync(self) -> None:
        check(lib().naiwa_event_sync(self.handle), "event_sync")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        check(lib().naiwa_event_elapsed_ms(C.byref(ms), self.handle, end.handle), "elapsed")
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            lib().naiwa_event_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass
