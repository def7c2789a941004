"""Minimal ctypes access to the HIP runtime that libarm_ai_amd.so is bound to.

Plumbing for tests and the benchmark (device buffers, copies, events, stream
capture into graphs).  The runtime is looked up by its soname *after* the
product library is loaded, so both always talk to the same HIP runtime
instance (a second copy of libamdhip64 in the process -- e.g. one bundled
with another package -- would own separate device state).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

_hip = None

H2D, D2H, D2D = 1, 2, 3
CAPTURE_MODE_RELAXED = 2


def rt() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _lib.load()  # binds libamdhip64.so.7 first
        h = ctypes.CDLL("libamdhip64.so.7")
        P, I, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        sig = {
            "hipMalloc": [ctypes.POINTER(P), SZ],
            "hipFree": [P],
            "hipMemcpy": [P, P, SZ, I],
            "hipMemcpyAsync": [P, P, SZ, I, P],
            "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [P],
            "hipEventCreate": [ctypes.POINTER(P)],
            "hipEventDestroy": [P],
            "hipEventRecord": [P, P],
            "hipEventSynchronize": [P],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), P, P],
            "hipStreamBeginCapture": [P, I],
            "hipStreamEndCapture": [P, ctypes.POINTER(P)],
            "hipGraphInstantiate": [ctypes.POINTER(P), P, P, P, SZ],
            "hipGraphUpload": [P, P],
            "hipGraphLaunch": [P, P],
            "hipGraphExecDestroy": [P],
            "hipGraphDestroy": [P],
            "hipGetErrorString": [I],
        }
        for name, args in sig.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = ctypes.c_char_p if name == "hipGetErrorString" else I
        _hip = h
    return _hip


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise RuntimeError(f"HIP error {rc} ({rt().hipGetErrorString(rc).decode()}) {what}")


class DeviceBuffer:
    """hipMalloc'd bytes; freed on close()/GC."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(rt().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    def upload(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(rt().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "H2D")
        return self

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(rt().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "D2H")
        return out

    def close(self) -> None:
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def to_device(a: np.ndarray) -> DeviceBuffer:
    a = np.ascontiguousarray(a)
    return DeviceBuffer(a.nbytes).upload(a)


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(rt().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.h = e.value

    def record(self, stream: int) -> None:
        check(rt().hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self) -> None:
        check(rt().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(rt().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            rt().hipEventDestroy(self.h)
        except Exception:
            pass


class Graph:
    """Captures the work enqueued on `stream` by fn() and replays it."""

    def __init__(self, stream: int, fn):
        h = rt()
        check(h.hipStreamBeginCapture(stream, CAPTURE_MODE_RELAXED), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            rc = h.hipStreamEndCapture(stream, ctypes.byref(g))
        check(rc, "hipStreamEndCapture")
        self.graph = g.value
        ex = ctypes.c_void_p()
        check(h.hipGraphInstantiate(ctypes.byref(ex), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = ex.value
        self.stream = stream
        check(h.hipGraphUpload(self.exec, stream), "hipGraphUpload")

    def launch(self) -> None:
        check(rt().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def __del__(self):
        try:
            rt().hipGraphExecDestroy(self.exec)
            rt().hipGraphDestroy(self.graph)
        except Exception:
            pass


def synchronize() -> None:
    check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")
