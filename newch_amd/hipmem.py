"""Device buffers and timing for callers of the kernel layer, over the HIP runtime libnc.so uses.

The runtime is reached by soname after newch_amd/libnc.so is loaded, so this module and the
library always share one HIP runtime in the process (a second runtime -- e.g. one bundled inside
another Python package and loaded later -- would not see the device).

    buf = DeviceBuffer.from_numpy(x)       # hipMalloc + upload
    y = DeviceBuffer.empty(x.nbytes)
    kernels.unary_fwd("gelu", buf.ptr, y.ptr, x.size)
    out = y.to_numpy(np.float32, x.shape)  # synchronising download
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_size_t, c_void_p

import numpy as np

from . import abi

H2D, D2H, D2D = 1, 2, 3

_rt = None


def runtime() -> ctypes.CDLL:
    global _rt
    if _rt is None:
        ctypes.CDLL(str(abi.LIB_PATH))              # loads the runtime libnc.so is linked against
        rt = ctypes.CDLL("libamdhip64.so.7")        # ... and resolves to that same object
        sig = {
            "hipMalloc": (c_int, [POINTER(c_void_p), c_size_t]),
            "hipFree": (c_int, [c_void_p]),
            "hipMemcpy": (c_int, [c_void_p, c_void_p, c_size_t, c_int]),
            "hipMemcpyAsync": (c_int, [c_void_p, c_void_p, c_size_t, c_int, c_void_p]),
            "hipMemset": (c_int, [c_void_p, c_int, c_size_t]),
            "hipDeviceSynchronize": (c_int, []),
            "hipStreamCreate": (c_int, [POINTER(c_void_p)]),
            "hipStreamDestroy": (c_int, [c_void_p]),
            "hipStreamSynchronize": (c_int, [c_void_p]),
            "hipEventCreate": (c_int, [POINTER(c_void_p)]),
            "hipEventDestroy": (c_int, [c_void_p]),
            "hipEventRecord": (c_int, [c_void_p, c_void_p]),
            "hipEventSynchronize": (c_int, [c_void_p]),
            "hipEventElapsedTime": (c_int, [POINTER(c_float), c_void_p, c_void_p]),
            "hipGetErrorString": (c_char_p, [c_int]),
            "hipGetDeviceCount": (c_int, [POINTER(c_int)]),
            "hipSetDevice": (c_int, [c_int]),
            "hipMemGetInfo": (c_int, [POINTER(c_size_t), POINTER(c_size_t)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(rt, name)
            fn.restype, fn.argtypes = res, args
        _rt = rt
    return _rt


class HipError(RuntimeError):
    pass


def check(rc: int, what: str):
    if rc != 0:
        raise HipError(f"{what}: {runtime().hipGetErrorString(rc).decode()} ({rc})")


def device_count() -> int:
    n = c_int(0)
    return n.value if runtime().hipGetDeviceCount(byref(n)) == 0 else 0


def synchronize():
    check(runtime().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info() -> tuple[int, int]:
    free, total = c_size_t(), c_size_t()
    check(runtime().hipMemGetInfo(byref(free), byref(total)), "hipMemGetInfo")
    return free.value, total.value


class DeviceBuffer:
    """An owned device allocation; `ptr` is its address as an int."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = c_void_p()
        check(runtime().hipMalloc(byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def empty(cls, nbytes: int) -> "DeviceBuffer":
        return cls(nbytes)

    @classmethod
    def from_numpy(cls, a: np.ndarray, pad: int = 0) -> "DeviceBuffer":
        """Uploads a (made contiguous) array; `pad` extra bytes are allocated in front (for offset tests)."""
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes + pad)
        if a.nbytes:
            check(runtime().hipMemcpy(c_void_p(buf.ptr + pad), a.ctypes.data_as(c_void_p), a.nbytes, H2D), "upload")
        return buf

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(runtime().hipMemcpy(c_void_p(self.ptr + offset), a.ctypes.data_as(c_void_p), a.nbytes, H2D), "upload")

    def to_numpy(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert offset + out.nbytes <= self.nbytes
        if out.nbytes:
            check(runtime().hipMemcpy(out.ctypes.data_as(c_void_p), c_void_p(self.ptr + offset), out.nbytes, D2H),
                  "download")
        return out

    def zero(self):
        check(runtime().hipMemset(c_void_p(self.ptr), 0, self.nbytes), "hipMemset")

    def free(self):
        if self.ptr:
            runtime().hipFree(c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = c_void_p()
        check(runtime().hipStreamCreate(byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self):
        check(runtime().hipStreamSynchronize(c_void_p(self.handle)), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.handle:
                runtime().hipStreamDestroy(c_void_p(self.handle))
        except Exception:
            pass


class Event:
    def __init__(self):
        e = c_void_p()
        check(runtime().hipEventCreate(byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream=None):
        check(runtime().hipEventRecord(c_void_p(self.handle), c_void_p(stream) if stream else None), "hipEventRecord")

    def synchronize(self):
        check(runtime().hipEventSynchronize(c_void_p(self.handle)), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float()
        check(runtime().hipEventElapsedTime(byref(ms), c_void_p(self.handle), c_void_p(end.handle)),
              "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                runtime().hipEventDestroy(c_void_p(self.handle))
        except Exception:
            pass


__all__ = ["DeviceBuffer", "Stream", "Event", "device_count", "synchronize", "mem_info", "HipError"]
