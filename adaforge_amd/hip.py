"""Minimal HIP runtime plumbing over ctypes (device buffers, copies, streams, events).

The harness uses the same libamdhip64 the C-ABI library links, resolved after
that library is loaded, so both share one HIP runtime in the process.  (The
PyTorch wheel ships its own HIP runtime with the same soname; it is not used.)
"""
import ctypes

import numpy as np

from . import _native

_hip = None
H2D, D2H, D2D = 1, 2, 3


def rt():
    global _hip
    if _hip is None:
        _native.lib()  # bind the runtime the library resolved
        h = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
        P, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        h.hipMalloc.argtypes = [ctypes.POINTER(P), sz]
        h.hipFree.argtypes = [P]
        h.hipMemcpy.argtypes = [P, P, sz, i32]
        h.hipMemset.argtypes = [P, i32, sz]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamCreate.argtypes = [ctypes.POINTER(P)]
        h.hipStreamDestroy.argtypes = [P]
        h.hipStreamSynchronize.argtypes = [P]
        h.hipEventCreate.argtypes = [ctypes.POINTER(P)]
        h.hipEventDestroy.argtypes = [P]
        h.hipEventRecord.argtypes = [P, P]
        h.hipEventSynchronize.argtypes = [P]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), P, P]
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [i32]
        h.hipGetDeviceCount.argtypes = [ctypes.POINTER(i32)]
        h.hipStreamBeginCapture.argtypes = [P, i32]
        h.hipStreamEndCapture.argtypes = [P, ctypes.POINTER(P)]
        h.hipGraphInstantiate.argtypes = [ctypes.POINTER(P), P, P, P, sz]
        h.hipGraphLaunch.argtypes = [P, P]
        h.hipGraphExecDestroy.argtypes = [P]
        h.hipGraphDestroy.argtypes = [P]
        _hip = h
    return _hip


def ok(rc):
    if rc != 0:
        raise RuntimeError("HIP error: " + rt().hipGetErrorString(rc).decode())


def device_count():
    n = ctypes.c_int(0)
    if rt().hipGetDeviceCount(ctypes.byref(n)) != 0:
        return 0
    return n.value


def synchronize():
    ok(rt().hipDeviceSynchronize())


class Buffer:
    """A device allocation viewed as a typed array."""

    def __init__(self, shape, dtype=np.float32, zero=False):
        self.shape = tuple(np.atleast_1d(shape).tolist()) if not isinstance(shape, tuple) else shape
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        ok(rt().hipMalloc(ctypes.byref(p), max(self.nbytes, 16)))
        self.ptr = p.value
        if zero:
            ok(rt().hipMemset(self.ptr, 0, max(self.nbytes, 16)))

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.shape, a.dtype)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        ok(rt().hipMemcpy(self.ptr, a.ctypes.data, self.nbytes, H2D))

    def numpy(self):
        out = np.empty(self.shape, dtype=self.dtype)
        ok(rt().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H))
        return out

    def free(self):
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        ok(rt().hipStreamCreate(ctypes.byref(p)))
        self.handle = p.value

    def synchronize(self):
        ok(rt().hipStreamSynchronize(self.handle))

    def __del__(self):
        try:
            if self.handle:
                rt().hipStreamDestroy(self.handle)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        ok(rt().hipEventCreate(ctypes.byref(p)))
        self.handle = p.value

    def record(self, stream=None):
        ok(rt().hipEventRecord(self.handle, stream.handle if stream else None))

    def synchronize(self):
        ok(rt().hipEventSynchronize(self.handle))

    def elapsed_ms(self, end):
        t = ctypes.c_float()
        ok(rt().hipEventElapsedTime(ctypes.byref(t), self.handle, end.handle))
        return t.value

    def __del__(self):
        try:
            if self.handle:
                rt().hipEventDestroy(self.handle)
        except Exception:
            pass


class Graph:
    """The launches `enqueue()` makes on `stream`, captured once (stream capture, thread-local mode)
    and replayed with launch()."""

    def __init__(self, stream, enqueue):
        g, x = ctypes.c_void_p(), ctypes.c_void_p()
        ok(rt().hipStreamBeginCapture(stream.handle, 1))
        try:
            enqueue()
        finally:
            ok(rt().hipStreamEndCapture(stream.handle, ctypes.byref(g)))
        self.graph = g.value
        ok(rt().hipGraphInstantiate(ctypes.byref(x), self.graph, None, None, 0))
        self.exec = x.value

    def launch(self, stream):
        ok(rt().hipGraphLaunch(self.exec, stream.handle))

    def __del__(self):
        try:
            if self.exec:
                rt().hipGraphExecDestroy(self.exec)
            if self.graph:
                rt().hipGraphDestroy(self.graph)
        except Exception:
            pass
