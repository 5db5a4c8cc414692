"""Minimal ctypes binding of the HIP runtime that libfaie2fn.so itself links (/opt/rocm libamdhip64.so.7).

Device memory, streams, events and graphs for the Python side (tests, smoke, bench).  It exists because PyTorch
wheels bundle a HIP runtime of their own: two HIP runtimes in one process do not share devices, so the callers of
libfaie2fn.so's device entry points allocate and time through this one instead.
"""

import ctypes as C

import numpy as np

_H2D, _D2H, _D2D = 1, 2, 3
_lib = None


def lib():
    global _lib
    if _lib is None:
        for name in ("libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so.7", "libamdhip64.so"):
            try:
                _lib = C.CDLL(name)
                break
            except OSError:
                continue
        if _lib is None:
            raise RuntimeError("HIP runtime libamdhip64.so.7 not found")
        L = _lib
        vp, sz = C.c_void_p, C.c_size_t
        L.hipGetErrorString.restype = C.c_char_p
        L.hipMalloc.argtypes = [C.POINTER(vp), sz]
        L.hipFree.argtypes = [vp]
        L.hipMemcpy.argtypes = [vp, vp, sz, C.c_int]
        L.hipMemcpyAsync.argtypes = [vp, vp, sz, C.c_int, vp]
        L.hipMemsetAsync.argtypes = [vp, C.c_int, sz, vp]
        L.hipStreamCreate.argtypes = [C.POINTER(vp)]
        L.hipStreamDestroy.argtypes = [vp]
        L.hipStreamSynchronize.argtypes = [vp]
        L.hipEventCreate.argtypes = [C.POINTER(vp)]
        L.hipEventDestroy.argtypes = [vp]
        L.hipEventRecord.argtypes = [vp, vp]
        L.hipEventSynchronize.argtypes = [vp]
        L.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        L.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        L.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        L.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, sz]
        L.hipGraphLaunch.argtypes = [vp, vp]
        L.hipGraphExecDestroy.argtypes = [vp]
        L.hipGraphDestroy.argtypes = [vp]
        L.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        L.hipSetDevice.argtypes = [C.c_int]
        L.hipMemGetInfo.argtypes = [C.POINTER(sz), C.POINTER(sz)]
    return _lib


def check(rc, what="hip"):
    if rc != 0:
        raise RuntimeError(f"{what} failed: {lib().hipGetErrorString(rc).decode()} ({rc})")


def device_count():
    n = C.c_int(0)
    rc = lib().hipGetDeviceCount(C.byref(n))
    return n.value if rc == 0 else 0


def sync():
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info():
    f, t = C.c_size_t(0), C.c_size_t(0)
    check(lib().hipMemGetInfo(C.byref(f), C.byref(t)), "hipMemGetInfo")
    return f.value, t.value


def htod(ptr, arr):
    """Copy a host array to device address ptr (synchronous)."""
    arr = np.ascontiguousarray(arr)
    check(lib().hipMemcpy(ptr, arr.ctypes.data, arr.nbytes, _H2D), "hipMemcpy H2D")


def dtoh(ptr, shape, dtype=np.float32):
    """Copy device address ptr into a new host array of shape/dtype (synchronous)."""
    out = np.empty(shape, dtype)
    check(lib().hipMemcpy(out.ctypes.data, ptr, out.nbytes, _D2H), "hipMemcpy D2H")
    return out


class Buf:
    """A device allocation of nbytes, freed with free() or on garbage collection."""

    def __init__(self, nbytes, dtype=np.float32, shape=None):
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = C.c_void_p()
        check(lib().hipMalloc(C.byref(p), max(1, self.nbytes)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def like(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes, arr.dtype, arr.shape)
        b.upload(arr)
        return b

    @classmethod
    def empty(cls, shape, dtype=np.float32):
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return cls(n, dtype, tuple(shape))

    def upload(self, arr, stream=None):
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        assert arr.nbytes <= self.nbytes
        check(lib().hipMemcpy(self.ptr, arr.ctypes.data, arr.nbytes, _H2D), "hipMemcpy H2D")

    def download(self, shape=None):
        shape = self.shape if shape is None else shape
        out = np.empty(shape, self.dtype)
        assert out.nbytes <= self.nbytes
        check(lib().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, _D2H), "hipMemcpy D2H")
        return out

    def zero(self, stream=None):
        check(lib().hipMemsetAsync(self.ptr, 0, self.nbytes, stream), "hipMemsetAsync")

    def copy_from(self, other, nbytes=None, stream=None):
        n = self.nbytes if nbytes is None else nbytes
        check(lib().hipMemcpyAsync(self.ptr, other.ptr, n, _D2D, stream), "hipMemcpyAsync D2D")

    def free(self):
        if getattr(self, "ptr", None):
            lib().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = C.c_void_p()
        check(lib().hipStreamCreate(C.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def sync(self):
        check(lib().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self):
        if self.handle:
            lib().hipStreamDestroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(lib().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream):
        check(lib().hipEventRecord(self.handle, stream.handle if isinstance(stream, Stream) else stream),
              "hipEventRecord")

    def sync(self):
        check(lib().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def ms_since(self, start):
        ms = C.c_float(0.0)
        check(lib().hipEventElapsedTime(C.byref(ms), start.handle, self.handle), "hipEventElapsedTime")
        return ms.value


class Graph:
    """Stream capture of a callable into a hipGraph, replayed with launch()."""

    def __init__(self, stream, fn):
        g = C.c_void_p()
        check(lib().hipStreamBeginCapture(stream.handle, 0), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            rc = lib().hipStreamEndCapture(stream.handle, C.byref(g))
        check(rc, "hipStreamEndCapture")
        self.graph = g.value
        ge = C.c_void_p()
        check(lib().hipGraphInstantiate(C.byref(ge), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = ge.value
        self.stream = stream

    def launch(self):
        check(lib().hipGraphLaunch(self.exec, self.stream.handle), "hipGraphLaunch")

    def destroy(self):
        if self.exec:
            lib().hipGraphExecDestroy(self.exec)
            lib().hipGraphDestroy(self.graph)
            self.exec = None
