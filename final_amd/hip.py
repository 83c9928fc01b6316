"""Minimal HIP runtime plumbing over ctypes: device buffers, streams, events.

Tests and the benchmark drive the C-ABI with these instead of a framework so a
GPU process holds exactly one HIP runtime (the one libfinal_amd_moe.so links).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native

_hip = None
_vp = ctypes.c_void_p

hipMemcpyHostToDevice = 1
hipMemcpyDeviceToHost = 2
hipMemcpyDeviceToDevice = 3


def rt() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _native.lib()  # loads libamdhip64 as its dependency first
        H = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
        H.hipMalloc.argtypes = [ctypes.POINTER(_vp), ctypes.c_size_t]
        H.hipFree.argtypes = [_vp]
        H.hipMemcpy.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.c_int]
        H.hipMemcpyAsync.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.c_int, _vp]
        H.hipMemsetAsync.argtypes = [_vp, ctypes.c_int, ctypes.c_size_t, _vp]
        H.hipStreamCreate.argtypes = [ctypes.POINTER(_vp)]
        H.hipStreamDestroy.argtypes = [_vp]
        H.hipStreamSynchronize.argtypes = [_vp]
        H.hipEventCreate.argtypes = [ctypes.POINTER(_vp)]
        H.hipEventDestroy.argtypes = [_vp]
        H.hipEventRecord.argtypes = [_vp, _vp]
        H.hipEventSynchronize.argtypes = [_vp]
        H.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), _vp, _vp]
        H.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        H.hipSetDevice.argtypes = [ctypes.c_int]
        H.hipGetErrorString.argtypes = [ctypes.c_int]
        H.hipGetErrorString.restype = ctypes.c_char_p
        H.hipDeviceGetAttribute.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        _hip = H
    return _hip


def _ck(err: int, what: str) -> None:
    if err != 0:
        msg = rt().hipGetErrorString(err).decode()
        raise RuntimeError(f"{what}: HIP error {err} ({msg})")


def device_count() -> int:
    n = ctypes.c_int(0)
    err = rt().hipGetDeviceCount(ctypes.byref(n))
    return int(n.value) if err == 0 else 0


def synchronize() -> None:
    _ck(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")


def copy_device(dst: "DeviceArray", src: "DeviceArray") -> None:
    assert dst.nbytes == src.nbytes
    _ck(rt().hipMemcpy(dst.handle, src.handle, dst.nbytes, hipMemcpyDeviceToDevice),
        "hipMemcpy D2D")


class Stream:
    def __init__(self):
        self.handle = _vp()
        _ck(rt().hipStreamCreate(ctypes.byref(self.handle)), "hipStreamCreate")

    @property
    def ptr(self):
        return self.handle.value

    def synchronize(self) -> None:
        _ck(rt().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def close(self) -> None:
        if self.handle:
            rt().hipStreamDestroy(self.handle)
            self.handle = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        self.handle = _vp()
        _ck(rt().hipEventCreate(ctypes.byref(self.handle)), "hipEventCreate")

    def record(self, stream=None) -> None:
        _ck(rt().hipEventRecord(self.handle, stream.handle if stream else None), "hipEventRecord")

    def synchronize(self) -> None:
        _ck(rt().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        v = ctypes.c_float(0)
        _ck(rt().hipEventElapsedTime(ctypes.byref(v), self.handle, end.handle), "hipEventElapsedTime")
        return float(v.value)

    def __del__(self):
        try:
            if self.handle:
                rt().hipEventDestroy(self.handle)
        except Exception:
            pass


class DeviceArray:
    """A hipMalloc'd buffer with numpy-shaped upload/download."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.handle = _vp()
        _ck(rt().hipMalloc(ctypes.byref(self.handle), max(self.nbytes, 16)), "hipMalloc")

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    @property
    def ptr(self) -> int:
        return self.handle.value

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        _ck(rt().hipMemcpy(self.handle, a.ctypes.data, self.nbytes, hipMemcpyHostToDevice), "hipMemcpy H2D")

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        _ck(rt().hipMemcpy(out.ctypes.data, self.handle, self.nbytes, hipMemcpyDeviceToHost), "hipMemcpy D2H")
        return out

    def fill_async(self, byte: int, stream: Stream | None = None) -> None:
        _ck(rt().hipMemsetAsync(self.handle, byte, self.nbytes, stream.handle if stream else None),
            "hipMemsetAsync")

    def free(self) -> None:
        if self.handle:
            rt().hipFree(self.handle)
            self.handle = _vp()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
