"""Minimal HIP runtime access (device memory, copies, events) for the Python
side of spq4k, over the same libamdhip64 instance that libspq4k.so links.

torch wheels bundle their own HIP runtime; loading both into one process
gives two runtimes fighting over the device. The Python tools of this path
therefore never import torch in a process that uses libspq4k, and manage
device buffers through this module instead.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

_hip = None

H2D, D2H, D2D = 1, 2, 3


def _lib():
    global _hip
    if _hip is not None:
        return _hip
    from . import load_library
    load_library()  # binds libamdhip64.so.7 from /opt/rocm
    h = C.CDLL("libamdhip64.so.7")
    V, I, S = C.c_void_p, C.c_int, C.c_size_t
    for name, res, args in (
        ("hipMalloc", I, [C.POINTER(V), S]),
        ("hipFree", I, [V]),
        ("hipMemcpy", I, [V, V, S, I]),
        ("hipMemcpyAsync", I, [V, V, S, I, V]),
        ("hipMemset", I, [V, I, S]),
        ("hipMemsetAsync", I, [V, I, S, V]),
        ("hipDeviceSynchronize", I, []),
        ("hipStreamSynchronize", I, [V]),
        ("hipEventCreate", I, [C.POINTER(V)]),
        ("hipEventDestroy", I, [V]),
        ("hipEventRecord", I, [V, V]),
        ("hipEventSynchronize", I, [V]),
        ("hipEventElapsedTime", I, [C.POINTER(C.c_float), V, V]),
        ("hipGetErrorString", C.c_char_p, [I]),
        ("hipGetDeviceCount", I, [C.POINTER(I)]),
        ("hipMemGetInfo", I, [C.POINTER(S), C.POINTER(S)]),
        ("hipStreamBeginCapture", I, [V, I]),
        ("hipStreamEndCapture", I, [V, C.POINTER(V)]),
        ("hipGraphInstantiate", I, [C.POINTER(V), V, V, V, S]),
        ("hipGraphLaunch", I, [V, V]),
        ("hipGraphExecDestroy", I, [V]),
        ("hipGraphDestroy", I, [V]),
    ):
        f = getattr(h, name)
        f.restype = res
        f.argtypes = args
    _hip = h
    return h


def check(rc, what):
    if rc != 0:
        msg = _lib().hipGetErrorString(rc)
        raise RuntimeError(f"{what}: HIP error {rc} {msg.decode() if msg else ''}")


def device_count() -> int:
    n = C.c_int(0)
    if _lib().hipGetDeviceCount(C.byref(n)) != 0:
        return 0
    return n.value


def mem_info():
    f, t = C.c_size_t(), C.c_size_t()
    check(_lib().hipMemGetInfo(C.byref(f), C.byref(t)), "hipMemGetInfo")
    return f.value, t.value


def synchronize():
    check(_lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def download(ptr: int, nbytes: int) -> np.ndarray:
    """nbytes of device memory at ptr, as uint8 (synchronous)."""
    out = np.empty(nbytes, np.uint8)
    if nbytes:
        check(_lib().hipMemcpy(out.ctypes.data, ptr, nbytes, D2H), "hipMemcpy D2H")
    return out


class DeviceArray:
    """A device allocation with a numpy dtype/shape (no arithmetic)."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        check(_lib().hipMalloc(C.byref(p), max(self.nbytes, 16)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.copy_from(a)
        return d

    def copy_from(self, a: np.ndarray):
        a = np.ascontiguousarray(a, self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        check(_lib().hipMemcpy(self.ptr, a.ctypes.data, self.nbytes, H2D), "hipMemcpy H2D")

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(_lib().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill_byte(self, value: int):
        check(_lib().hipMemset(self.ptr, value, self.nbytes), "hipMemset")

    def free(self):
        if self.ptr:
            _lib().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(_lib().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.h = e.value

    def record(self, stream=None):
        check(_lib().hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self):
        check(_lib().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(_lib().hipEventElapsedTime(C.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.h:
                _lib().hipEventDestroy(self.h)
        except Exception:
            pass


class Graph:
    """A HIP graph captured from the work enqueued on `stream` inside
    `with Graph.capture(stream) as g:`; replay with g.launch()."""

    CAPTURE_RELAXED = 2

    def __init__(self, stream):
        self.stream = stream
        self.graph = None
        self.exec = None

    @classmethod
    def capture(cls, stream):
        return cls(stream)

    def __enter__(self):
        check(_lib().hipStreamBeginCapture(self.stream, self.CAPTURE_RELAXED), "hipStreamBeginCapture")
        return self

    def __exit__(self, et, ev, tb):
        g = C.c_void_p()
        rc = _lib().hipStreamEndCapture(self.stream, C.byref(g))
        if et is not None:
            return False
        check(rc, "hipStreamEndCapture")
        self.graph = g.value
        e = C.c_void_p()
        check(_lib().hipGraphInstantiate(C.byref(e), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = e.value
        return False

    def launch(self):
        check(_lib().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def __del__(self):
        try:
            if self.exec:
                _lib().hipGraphExecDestroy(self.exec)
            if self.graph:
                _lib().hipGraphDestroy(self.graph)
        except Exception:
            pass
