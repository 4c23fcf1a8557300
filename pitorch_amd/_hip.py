"""Minimal ctypes access to the HIP runtime that libptmi itself links
(/opt/rocm), for device buffers in tests and the benchmark.

torch ships a second HIP runtime of its own; two runtimes in one process
do not share the device, so nothing here imports torch."""
import ctypes
import os

import numpy as np

from ._ffi import load_ptmi

_hip = None


def hip():
    global _hip
    if _hip is not None:
        return _hip
    load_ptmi()   # makes the runtime libptmi links resident first
    for name in ("libamdhip64.so.7", "libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            H = ctypes.CDLL(name, mode=ctypes.RTLD_GLOBAL)
            break
        except OSError:
            continue
    else:
        raise RuntimeError("libamdhip64 not found")
    vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    H.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
    H.hipFree.argtypes = [vp]
    H.hipMemcpy.argtypes = [vp, vp, sz, i]
    H.hipDeviceSynchronize.argtypes = []
    H.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
    H.hipEventRecord.argtypes = [vp, vp]
    H.hipEventSynchronize.argtypes = [vp]
    H.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
    H.hipEventDestroy.argtypes = [vp]
    H.hipStreamBeginCapture.argtypes = [vp, i]
    H.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    H.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, sz]
    H.hipGraphLaunch.argtypes = [vp, vp]
    H.hipGraphExecDestroy.argtypes = [vp]
    H.hipGraphDestroy.argtypes = [vp]
    _hip = H
    return H


H2D, D2H = 1, 2


class DeviceArray:
    """A hipMalloc'd float32/int32 buffer with host copy helpers."""

    def __init__(self, n, dtype=np.float32):
        self.n, self.dtype = int(n), np.dtype(dtype)
        p = ctypes.c_void_p()
        st = hip().hipMalloc(ctypes.byref(p), max(1, self.n * self.dtype.itemsize))
        if st != 0:
            raise MemoryError(f"hipMalloc failed ({st})")
        self.ptr = p.value

    @classmethod
    def from_host(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.size, a.dtype)
        d.upload(a)
        return d

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.size <= self.n
        assert hip().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D) == 0

    def download(self, n=None):
        out = np.empty(self.n if n is None else n, self.dtype)
        assert hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H) == 0
        return out

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        assert hip().hipEventCreate(ctypes.byref(p)) == 0
        self.h = p.value

    def record(self, stream):
        assert hip().hipEventRecord(self.h, stream) == 0

    def elapsed_ms(self, later):
        hip().hipEventSynchronize(later.h)
        ms = ctypes.c_float()
        assert hip().hipEventElapsedTime(ctypes.byref(ms), self.h, later.h) == 0
        return ms.value


class Graph:
    """Stream capture of whatever `fn()` enqueues on `stream`, replayable."""

    CAPTURE_THREAD_LOCAL = 1

    def __init__(self, stream, fn):
        H = hip()
        self.stream = stream
        assert H.hipStreamBeginCapture(stream, self.CAPTURE_THREAD_LOCAL) == 0
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            st = H.hipStreamEndCapture(stream, ctypes.byref(g))
        assert st == 0, f"hipStreamEndCapture failed ({st})"
        self.graph = g.value
        e = ctypes.c_void_p()
        assert H.hipGraphInstantiate(ctypes.byref(e), self.graph, None, None, 0) == 0
        self.exec = e.value

    def launch(self):
        assert hip().hipGraphLaunch(self.exec, self.stream) == 0

    def free(self):
        if self.exec:
            hip().hipGraphExecDestroy(self.exec)
            hip().hipGraphDestroy(self.graph)
            self.exec = self.graph = None
