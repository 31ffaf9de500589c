"""Minimal HIP runtime access through ctypes (device memory, copies, streams, events).

Plumbing for the tests and the benchmark: libtiermm.so takes plain device
pointers, and this module provides them without any framework.  Every call
checks its hipError_t and raises ``HipError``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
_hip = None

H2D, D2H, D2D = 1, 2, 3  # hipMemcpyKind


class HipError(RuntimeError):
    pass


def lib():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL(os.path.join(_ROCM, "lib", "libamdhip64.so"))
        _hip.hipGetErrorString.restype = ctypes.c_char_p
        _hip.hipGetErrorString.argtypes = [ctypes.c_int]
    return _hip


def check(err: int, what: str = "") -> None:
    if err != 0:
        msg = lib().hipGetErrorString(err).decode()
        raise HipError(f"{what}: hip error {err} ({msg})")


def device_count() -> int:
    n = ctypes.c_int(0)
    err = lib().hipGetDeviceCount(ctypes.byref(n))
    return n.value if err == 0 else 0


def set_device(d: int) -> None:
    check(lib().hipSetDevice(d), "hipSetDevice")


def synchronize() -> None:
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def attribute(attr: int, dev: int = 0) -> int:
    v = ctypes.c_int(0)
    check(lib().hipDeviceGetAttribute(ctypes.byref(v), attr, dev), "hipDeviceGetAttribute")
    return v.value


# hipDeviceAttribute_t values used by the benchmark
# (values of the ROCm 7 hip_runtime_api.h enum)
ATTR_CLOCK_RATE_KHZ = 5      # hipDeviceAttributeClockRate
ATTR_MEM_BUS_WIDTH = 59      # hipDeviceAttributeMemoryBusWidth
ATTR_MEM_CLOCK_KHZ = 60      # hipDeviceAttributeMemoryClockRate
ATTR_MULTIPROCESSORS = 63    # hipDeviceAttributeMultiprocessorCount


class DeviceBuffer:
    """Owned device allocation.  ``ptr`` is the raw device address (int)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().hipMalloc(ctypes.byref(p), ctypes.c_size_t(max(self.nbytes, 1))), f"hipMalloc({nbytes})")
        self.ptr = p.value

    def free(self) -> None:
        if self.ptr:
            check(lib().hipFree(ctypes.c_void_p(self.ptr)), "hipFree")
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, arr: np.ndarray, offset: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        check(lib().hipMemcpy(ctypes.c_void_p(self.ptr + offset), a.ctypes.data_as(ctypes.c_void_p),
                              ctypes.c_size_t(a.nbytes), H2D), "hipMemcpy H2D")
        return self

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        count = (self.nbytes - offset) // dt.itemsize if count is None else count
        out = np.empty(count, dtype=dt)
        check(lib().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr + offset),
                              ctypes.c_size_t(out.nbytes), D2H), "hipMemcpy D2H")
        return out

    def fill_bytes(self, value: int) -> None:
        check(lib().hipMemset(ctypes.c_void_p(self.ptr), ctypes.c_int(value), ctypes.c_size_t(self.nbytes)),
              "hipMemset")


def to_device(arr: np.ndarray) -> DeviceBuffer:
    a = np.ascontiguousarray(arr)
    return DeviceBuffer(a.nbytes).upload(a)


def copy_d2d(dst: int, src: int, nbytes: int) -> None:
    check(lib().hipMemcpy(ctypes.c_void_p(dst), ctypes.c_void_p(src), ctypes.c_size_t(nbytes), D2D), "hipMemcpy D2D")


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(lib().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        check(lib().hipStreamSynchronize(ctypes.c_void_p(self.handle)), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            check(lib().hipStreamDestroy(ctypes.c_void_p(self.handle)), "hipStreamDestroy")
            self.handle = None


class Graph:
    """The work ``record(stream)`` issues on ``stream``, captured once (relaxed mode) and
    instantiated; ``launch`` replays it on a stream."""

    def __init__(self, stream: Stream, record):
        h = lib()
        s = ctypes.c_void_p(stream.handle)
        check(h.hipStreamBeginCapture(s, 2), "hipStreamBeginCapture")  # hipStreamCaptureModeRelaxed
        g = ctypes.c_void_p()
        try:
            record(stream)
        finally:
            err = h.hipStreamEndCapture(s, ctypes.byref(g))
        check(err, "hipStreamEndCapture")
        self.graph = g.value
        ex = ctypes.c_void_p()
        check(h.hipGraphInstantiate(ctypes.byref(ex), ctypes.c_void_p(self.graph), None, None, ctypes.c_size_t(0)),
              "hipGraphInstantiate")
        self.exec = ex.value

    def launch(self, stream: Stream) -> None:
        check(lib().hipGraphLaunch(ctypes.c_void_p(self.exec), ctypes.c_void_p(stream.handle)), "hipGraphLaunch")

    def destroy(self) -> None:
        if self.exec:
            check(lib().hipGraphExecDestroy(ctypes.c_void_p(self.exec)), "hipGraphExecDestroy")
            self.exec = None
        if self.graph:
            check(lib().hipGraphDestroy(ctypes.c_void_p(self.graph)), "hipGraphDestroy")
            self.graph = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(lib().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream | None = None) -> None:
        s = ctypes.c_void_p(stream.handle if stream is not None else None)
        check(lib().hipEventRecord(ctypes.c_void_p(self.handle), s), "hipEventRecord")

    def synchronize(self) -> None:
        check(lib().hipEventSynchronize(ctypes.c_void_p(self.handle)), "hipEventSynchronize")

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float(0)
        check(lib().hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(self.handle), ctypes.c_void_p(later.handle)),
              "hipEventElapsedTime")
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            check(lib().hipEventDestroy(ctypes.c_void_p(self.handle)), "hipEventDestroy")
            self.handle = None
