"""Minimal HIP runtime access through ctypes: device memory, copies, streams
and events.

This uses the same libamdhip64 that libswiftllm_hip.so links against (it is
loaded by SONAME after the library), so pointers and streams handed to the
library belong to its runtime. Nothing here imports torch.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np

from . import _lib

_HIP: Optional[ctypes.CDLL] = None

HIP_MEMCPY_H2D = 1
HIP_MEMCPY_D2H = 2
HIP_MEMCPY_D2D = 3


class HipError(RuntimeError):
    pass


def hip() -> ctypes.CDLL:
    """The HIP runtime library used by libswiftllm_hip.so."""
    global _HIP
    if _HIP is None:
        _lib.lib()  # loads libamdhip64 as a dependency first
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [ctypes.c_int]
        vp = ctypes.c_void_p
        for name, args in {
            "hipMalloc": [ctypes.POINTER(vp), ctypes.c_size_t],
            "hipFree": [vp],
            "hipMemcpy": [vp, vp, ctypes.c_size_t, ctypes.c_int],
            "hipMemcpyAsync": [vp, vp, ctypes.c_size_t, ctypes.c_int, vp],
            "hipMemset": [vp, ctypes.c_int, ctypes.c_size_t],
            "hipDeviceSynchronize": [],
            "hipStreamCreate": [ctypes.POINTER(vp)],
            "hipStreamDestroy": [vp],
            "hipStreamSynchronize": [vp],
            "hipEventCreate": [ctypes.POINTER(vp)],
            "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
            "hipGetDeviceCount": [ctypes.POINTER(ctypes.c_int)],
            "hipSetDevice": [ctypes.c_int],
            "hipDeviceGetAttribute": [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int],
            "hipMemGetInfo": [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
            "hipHostMalloc": [ctypes.POINTER(vp), ctypes.c_size_t, ctypes.c_uint],
            "hipHostFree": [vp],
            "hipStreamBeginCapture": [vp, ctypes.c_int],
            "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
            "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t],
            "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp],
            "hipGraphDestroy": [vp],
        }.items():
            fn = getattr(h, name)
            fn.restype = ctypes.c_int
            fn.argtypes = args
        _HIP = h
    return _HIP


def check(err: int, what: str) -> None:
    if err != 0:
        msg = hip().hipGetErrorString(err).decode()
        raise HipError(f"{what}: HIP error {err}: {msg}")


def device_count() -> int:
    n = ctypes.c_int(0)
    err = hip().hipGetDeviceCount(ctypes.byref(n))
    return n.value if err == 0 else 0


def synchronize() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


def cu_count(device: int = 0) -> int:
    v = ctypes.c_int(0)
    # hipDeviceAttributeMultiprocessorCount
    check(hip().hipDeviceGetAttribute(ctypes.byref(v), 63, device), "hipDeviceGetAttribute")
    return v.value


class DeviceArray:
    """A device allocation with a numpy-like dtype and shape."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in np.atleast_1d(shape)) if np.ndim(shape) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self._ptr = p.value
        self._hip = hip()

    @property
    def ptr(self) -> int:
        return self._ptr

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = cls(arr.shape, arr.dtype)
        d.upload(arr)
        return d

    @classmethod
    def zeros(cls, shape, dtype) -> "DeviceArray":
        d = cls(shape, dtype)
        d.fill_zero()
        return d

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: {arr.nbytes} != {self.nbytes}")
        check(hip().hipMemcpy(self._ptr, arr.ctypes.data, self.nbytes, HIP_MEMCPY_H2D), "hipMemcpy H2D")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(hip().hipMemcpy(out.ctypes.data, self._ptr, self.nbytes, HIP_MEMCPY_D2H), "hipMemcpy D2H")
        return out

    def _span(self, offset: int, nbytes: int) -> int:
        if offset < 0 or nbytes < 0 or offset + nbytes > self.nbytes:
            raise ValueError(f"bytes [{offset}, {offset + nbytes}) outside a {self.nbytes}-byte array")
        return self._ptr + offset

    def upload_at(self, offset: int, arr: np.ndarray) -> None:
        """Copies arr's bytes to this array at byte `offset` (a slice of a
        large allocation, e.g. a few blocks of a KV pool)."""
        arr = np.ascontiguousarray(arr)
        check(hip().hipMemcpy(self._span(offset, arr.nbytes), arr.ctypes.data, arr.nbytes,
                              HIP_MEMCPY_H2D), "hipMemcpy H2D")

    def download_at(self, offset: int, shape, dtype) -> np.ndarray:
        """The bytes at byte `offset` as a host array of shape and dtype."""
        out = np.empty(shape, dtype=dtype)
        check(hip().hipMemcpy(out.ctypes.data, self._span(offset, out.nbytes), out.nbytes,
                              HIP_MEMCPY_D2H), "hipMemcpy D2H")
        return out

    def fill_zero(self) -> None:
        check(hip().hipMemset(self._ptr, 0, self.nbytes), "hipMemset")

    def fill_byte(self, value: int) -> None:
        check(hip().hipMemset(self._ptr, int(value), self.nbytes), "hipMemset")

    def free(self) -> None:
        if self._ptr:
            self._hip.hipFree(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HostArray:
    """Pinned host memory (hipHostMalloc) that kernels can address directly,
    with a numpy view of it."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in np.atleast_1d(shape)) if np.ndim(shape) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(hip().hipHostMalloc(ctypes.byref(p), max(self.nbytes, 1), 0),
              f"hipHostMalloc({self.nbytes})")
        self._ptr = p.value
        self._hip = hip()

    @property
    def ptr(self) -> int:
        return self._ptr

    def array(self) -> np.ndarray:
        """numpy view of the pinned buffer (valid while this object lives)."""
        buf = (ctypes.c_uint8 * max(self.nbytes, 1)).from_address(self._ptr)
        return np.frombuffer(buf, dtype=np.uint8, count=self.nbytes).view(self.dtype).reshape(self.shape)

    def free(self) -> None:
        if self._ptr:
            self._hip.hipHostFree(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(hip().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        check(hip().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.handle:
                hip().hipStreamDestroy(self.handle)
        except Exception:
            pass


class Graph:
    """A HIP graph of the work that `enqueue()` puts on `stream`, captured
    once and replayed with launch(). Buffers must exist before the capture:
    allocation and synchronous copies cannot be captured."""

    _CAPTURE_THREAD_LOCAL = 1

    def __init__(self, stream: Stream, enqueue) -> None:
        h = hip()
        check(h.hipStreamBeginCapture(stream.handle, self._CAPTURE_THREAD_LOCAL),
              "hipStreamBeginCapture")
        g = ctypes.c_void_p()
        try:
            enqueue()
        finally:
            end = h.hipStreamEndCapture(stream.handle, ctypes.byref(g))
        check(end, "hipStreamEndCapture")
        self._graph = g.value
        ex = ctypes.c_void_p()
        check(h.hipGraphInstantiate(ctypes.byref(ex), self._graph, None, None, 0),
              "hipGraphInstantiate")
        self._exec = ex.value
        self._hip = h

    def launch(self, stream: Stream) -> None:
        check(self._hip.hipGraphLaunch(self._exec, stream.handle), "hipGraphLaunch")

    def __del__(self):
        try:
            if getattr(self, "_exec", None):
                self._hip.hipGraphExecDestroy(self._exec)
            if getattr(self, "_graph", None):
                self._hip.hipGraphDestroy(self._graph)
        except Exception:
            pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Optional[Stream] = None) -> None:
        check(hip().hipEventRecord(self.handle, stream.handle if stream else None), "hipEventRecord")

    def synchronize(self) -> None:
        check(hip().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0.0)
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                hip().hipEventDestroy(self.handle)
        except Exception:
            pass
