"""Device buffers, streams and events from the HIP runtime the library links.

librusticide_hip.so links ROCm's libamdhip64; this module binds the same
runtime with ctypes for what callers of the device-pointer entry points need
(allocations, copies, events). PyTorch ships a second HIP runtime of its own,
and two runtimes in one process do not share the GPU, so nothing here
imports torch.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import lib as _rh_lib

_hip = None


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _rh_lib()  # load librusticide_hip.so first: it pins the runtime
        H = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
        P, S = ctypes.c_void_p, ctypes.c_size_t
        H.hipMalloc.argtypes = [ctypes.POINTER(P), S]
        H.hipFree.argtypes = [P]
        H.hipMemcpy.argtypes = [P, P, S, ctypes.c_int]
        H.hipMemset.argtypes = [P, ctypes.c_int, S]
        H.hipDeviceSynchronize.argtypes = []
        H.hipStreamSynchronize.argtypes = [P]
        H.hipEventCreate.argtypes = [ctypes.POINTER(P)]
        H.hipEventDestroy.argtypes = [P]
        H.hipEventRecord.argtypes = [P, P]
        H.hipEventSynchronize.argtypes = [P]
        H.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), P, P]
        H.hipHostMalloc.argtypes = [ctypes.POINTER(P), S, ctypes.c_uint]
        H.hipHostFree.argtypes = [P]
        H.hipGetErrorString.argtypes = [ctypes.c_int]
        H.hipGetErrorString.restype = ctypes.c_char_p
        _hip = H
    return _hip


def check(err: int, what: str = "") -> None:
    if err != 0:
        raise RuntimeError(f"HIP error {err} ({hip().hipGetErrorString(err).decode()}) in {what}")


H2D, D2H, D2D = 1, 2, 3


class DeviceArray:
    """A flat device allocation of `n` elements of `dtype`."""

    def __init__(self, n: int, dtype=np.float32):
        self.dtype = np.dtype(dtype)
        self.n = int(n)
        self.ptr = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(self.ptr), max(1, self.nbytes)), "hipMalloc")

    @property
    def nbytes(self) -> int:
        return self.n * self.dtype.itemsize

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.size, a.dtype)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.size <= self.n
        check(hip().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.n, self.dtype)
        check(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill_bytes(self, value: int) -> None:
        check(hip().hipMemset(self.ptr, value, self.nbytes), "hipMemset")

    # the interface rusticide_amd's device entry points read
    def data_ptr(self) -> int:
        return self.ptr.value or 0

    def numel(self) -> int:
        return self.n

    def free(self) -> None:
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        self.h = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(self.h)), "hipEventCreate")

    def record(self, stream: int) -> None:
        check(hip().hipEventRecord(self.h, ctypes.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            hip().hipEventDestroy(self.h)
        except Exception:
            pass


class PinnedHost:
    """`n` bytes of page-locked host memory (hipHostMalloc)."""

    def __init__(self, n: int):
        self.n = int(n)
        self.ptr = ctypes.c_void_p()
        check(hip().hipHostMalloc(ctypes.byref(self.ptr), max(1, self.n), 0), "hipHostMalloc")

    def free(self) -> None:
        if self.ptr:
            hip().hipHostFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
