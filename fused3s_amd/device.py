"""Device memory, streams and events through the C-ABI (no torch needed)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

F3S_OK = 0
STATUS_NAMES = {0: "F3S_OK", 1: "F3S_EINVAL", 2: "F3S_ENOMEM", 3: "F3S_EHIP",
                4: "F3S_ENODEV", 5: "F3S_EUNSUPPORTED", 6: "F3S_EDATA"}


class F3SError(RuntimeError):
    """A C-ABI call returned a non-zero f3s_status."""

    def __init__(self, status: int, where: str):
        lib = _lib.hip()
        detail = (lib.f3s_last_error() or b"").decode(errors="replace")
        self.status = status
        self.name = STATUS_NAMES.get(status, str(status))
        super().__init__(f"{where}: {self.name} ({detail})")


def check(status: int, where: str) -> None:
    if status != F3S_OK:
        raise F3SError(status, where)


def device_count() -> int:
    n = C.c_int32(0)
    check(_lib.hip().f3s_device_count(C.byref(n)), "f3s_device_count")
    return int(n.value)


def init() -> None:
    """Loads the library's GPU code now (f3s_init) instead of at first launch."""
    check(_lib.hip().f3s_init(), "f3s_init")


def device_name() -> str:
    buf = C.create_string_buffer(256)
    check(_lib.hip().f3s_device_name(buf, 256), "f3s_device_name")
    return buf.value.decode()


def synchronize(stream: "Stream | None" = None) -> None:
    check(_lib.hip().f3s_synchronize(stream.handle if stream else None), "f3s_synchronize")


class DeviceArray:
    """A typed device allocation made with f3s_malloc.

    ``DeviceArray.from_numpy(a)`` uploads; ``.numpy()`` downloads; ``.ptr`` is
    the raw device address passed to the C-ABI.
    """

    def __init__(self, shape, dtype, zero: bool = False):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(_lib.hip().f3s_malloc(C.byref(p), max(self.nbytes, 1)), "f3s_malloc")
        self._ptr = p.value
        if zero:
            self.zero()

    @property
    def ptr(self) -> int:
        return self._ptr

    @classmethod
    def from_numpy(cls, a: np.ndarray, stream: "Stream | None" = None) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a, stream)
        return d

    def upload(self, a: np.ndarray, stream: "Stream | None" = None) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError(f"upload of {a.nbytes} bytes into a {self.nbytes}-byte array")
        if self.nbytes:
            check(_lib.hip().f3s_memcpy_h2d(self._ptr, a.ctypes.data, self.nbytes,
                                            stream.handle if stream else None), "f3s_memcpy_h2d")

    def numpy(self, stream: "Stream | None" = None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            check(_lib.hip().f3s_memcpy_d2h(out.ctypes.data, self._ptr, self.nbytes,
                                            stream.handle if stream else None), "f3s_memcpy_d2h")
        return out

    def zero(self, stream: "Stream | None" = None) -> None:
        if self.nbytes:
            check(_lib.hip().f3s_memset(self._ptr, 0, self.nbytes,
                                        stream.handle if stream else None), "f3s_memset")

    def fill_bytes(self, value: int, stream: "Stream | None" = None) -> None:
        if self.nbytes:
            check(_lib.hip().f3s_memset(self._ptr, int(value), self.nbytes,
                                        stream.handle if stream else None), "f3s_memset")

    def free(self) -> None:
        if getattr(self, "_ptr", None):
            _lib.hip().f3s_free(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A non-blocking HIP stream (default priority)."""

    def __init__(self):
        h = C.c_void_p()
        check(_lib.hip().f3s_stream_create(C.byref(h)), "f3s_stream_create")
        self.handle = h.value

    def synchronize(self) -> None:
        synchronize(self)

    def __del__(self):
        try:
            if self.handle:
                _lib.hip().f3s_stream_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


class Event:
    def __init__(self):
        h = C.c_void_p()
        check(_lib.hip().f3s_event_create(C.byref(h)), "f3s_event_create")
        self.handle = h.value

    def record(self, stream: "Stream | None" = None) -> None:
        check(_lib.hip().f3s_event_record(self.handle, stream.handle if stream else None),
              "f3s_event_record")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        check(_lib.hip().f3s_event_elapsed_ms(self.handle, end.handle, C.byref(ms)),
              "f3s_event_elapsed_ms")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                _lib.hip().f3s_event_destroy(self.handle)
                self.handle = None
        except Exception:
            pass
