"""Minimal ctypes binding of the HIP runtime: device buffers, streams, events.

Tests and benchmarks use it to hand device pointers and a stream to the
*_dev entry points of libom_hip.so, and to time kernels with HIP events on
that same stream.  It binds the runtime by its soname, libamdhip64.so.7, so
it shares whatever copy libom_hip.so is linked against: one HIP runtime per
process.  (torch ships a second copy of the runtime; importing torch after
this module, or after libom_hip.so, would initialise that second copy and is
avoided in this package.)
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import gdn

_H = None
H2D, D2H, D2D = 1, 2, 3


def rt() -> C.CDLL:
    global _H
    if _H is None:
        gdn.lib()                                   # load libom_hip.so (and its runtime) first
        H = C.CDLL("libamdhip64.so.7")
        vp, sz = C.c_void_p, C.c_size_t
        H.hipMalloc.argtypes = [C.POINTER(vp), sz]
        H.hipFree.argtypes = [vp]
        H.hipMemcpy.argtypes = [vp, vp, sz, C.c_int]
        H.hipMemcpyAsync.argtypes = [vp, vp, sz, C.c_int, vp]
        H.hipMemsetAsync.argtypes = [vp, C.c_int, sz, vp]
        H.hipStreamCreateWithFlags.argtypes = [C.POINTER(vp), C.c_uint]
        H.hipStreamSynchronize.argtypes = [vp]
        H.hipStreamDestroy.argtypes = [vp]
        H.hipEventCreate.argtypes = [C.POINTER(vp)]
        H.hipEventRecord.argtypes = [vp, vp]
        H.hipEventSynchronize.argtypes = [vp]
        H.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        H.hipEventDestroy.argtypes = [vp]
        H.hipGetErrorString.restype = C.c_char_p
        H.hipGetErrorString.argtypes = [C.c_int]
        H.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        H.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        H.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, C.c_char_p, sz]
        H.hipGraphLaunch.argtypes = [vp, vp]
        H.hipGraphExecDestroy.argtypes = [vp]
        H.hipGraphDestroy.argtypes = [vp]
        H.hipGraphGetNodes.argtypes = [vp, vp, C.POINTER(sz)]
        _H = H
    return _H


def ok(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"HIP error {rc}: {rt().hipGetErrorString(rc).decode()}")


def device_synchronize() -> None:
    ok(rt().hipDeviceSynchronize())


class Buffer:
    """A device allocation of nbytes (freed on close / garbage collection)."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        ok(rt().hipMalloc(C.byref(p), max(int(nbytes), 16)))
        self.ptr, self.nbytes = p.value, int(nbytes)

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "Buffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        ok(rt().hipMemcpy(b.ptr, a.ctypes.data, a.nbytes, H2D))
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        ok(rt().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, H2D))

    def numpy(self, shape, dtype=np.float32, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert offset + out.nbytes <= self.nbytes
        ok(rt().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, D2H))
        return out

    def at(self, offset_bytes: int) -> int:
        return self.ptr + int(offset_bytes)

    def data_ptr(self) -> int:
        return self.ptr

    def close(self) -> None:
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    """A non-blocking stream at the default priority."""

    def __init__(self):
        s = C.c_void_p()
        ok(rt().hipStreamCreateWithFlags(C.byref(s), 1))
        self.cuda_stream = s.value

    def synchronize(self) -> None:
        ok(rt().hipStreamSynchronize(self.cuda_stream))


class Event:
    def __init__(self):
        e = C.c_void_p()
        ok(rt().hipEventCreate(C.byref(e)))
        self.h = e.value

    def record(self, stream: Stream | None) -> None:
        ok(rt().hipEventRecord(self.h, stream.cuda_stream if stream else None))

    def synchronize(self) -> None:
        ok(rt().hipEventSynchronize(self.h))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        ok(rt().hipEventElapsedTime(C.byref(ms), self.h, end.h))
        return ms.value


class Graph:
    """Work enqueued on one stream by a Python callable, captured once into
    a HIP graph (hipStreamCaptureModeThreadLocal) and replayed with
    launch().  The callable must only enqueue kernels on that stream: no
    allocation, no synchronisation, no memset nodes."""

    def __init__(self, stream: Stream, fn):
        H = rt()
        ok(H.hipStreamBeginCapture(stream.cuda_stream, 1))
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = H.hipStreamEndCapture(stream.cuda_stream, C.byref(g))
        ok(rc)
        self.graph = g.value
        n = C.c_size_t(0)
        ok(H.hipGraphGetNodes(self.graph, None, C.byref(n)))
        self.nodes = n.value
        e = C.c_void_p()
        ok(H.hipGraphInstantiate(C.byref(e), self.graph, None, None, 0))
        self.exec = e.value
        self.stream = stream

    def launch(self) -> None:
        ok(rt().hipGraphLaunch(self.exec, self.stream.cuda_stream))

    def close(self) -> None:
        if self.exec:
            rt().hipGraphExecDestroy(self.exec)
            rt().hipGraphDestroy(self.graph)
            self.exec = self.graph = None
