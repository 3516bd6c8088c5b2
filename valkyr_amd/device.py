"""Device memory, streams and events over the C ABI (no framework needed)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib

BF16 = "bf16"


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


class DeviceBuffer:
    """A hipMalloc'd buffer; freed when the object is collected."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().vkh_malloc(C.byref(p), max(1, self.nbytes)))
        self._p = p

    @property
    def ptr(self) -> C.c_void_p:
        return self._p

    @property
    def addr(self) -> int:
        return self._p.value

    def offset(self, nbytes: int) -> C.c_void_p:
        return C.c_void_p(self._p.value + int(nbytes))

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            check(lib().vkh_memcpy_h2d(b.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes))
        return b

    @classmethod
    def zeros(cls, nbytes: int) -> "DeviceBuffer":
        b = cls(nbytes)
        check(lib().vkh_memset(b.ptr, 0, max(1, b.nbytes)))
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().vkh_memcpy_h2d(self.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes))

    def to_numpy(self, dtype=np.float32, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype)
        if n:
            check(lib().vkh_memcpy_d2h(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes))
        return out

    def fill_zero(self) -> None:
        check(lib().vkh_memset(self.ptr, 0, max(1, self.nbytes)))

    def __del__(self):
        p = getattr(self, "_p", None)
        if p is not None and p.value:
            try:
                lib().vkh_free(p)
            except Exception:
                pass
            self._p = C.c_void_p()


class Stream:
    def __init__(self):
        s = C.c_void_p()
        check(lib().vkh_stream_create(C.byref(s)))
        self.handle = s

    def synchronize(self) -> None:
        check(lib().vkh_stream_synchronize(self.handle))

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                lib().vkh_stream_destroy(h)
            except Exception:
                pass
            self.handle = C.c_void_p()


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(lib().vkh_event_create(C.byref(e)))
        self.handle = e

    def record(self, stream=None) -> None:
        check(lib().vkh_event_record(self.handle, stream.handle if stream else None))

    def synchronize(self) -> None:
        check(lib().vkh_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(lib().vkh_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                lib().vkh_event_destroy(h)
            except Exception:
                pass
            self.handle = C.c_void_p()


def synchronize() -> None:
    check(lib().vkh_device_synchronize())
