"""Device buffers for the GPU tests, allocated and copied through the HIP runtime that libqne.so
itself links (/opt/rocm's libamdhip64.so.7, bound when conftest loads libqne before anything else).
The tests therefore run the library on the product's runtime; no second HIP runtime (torch's
bundled one) is loaded into a GPU test process."""
from __future__ import annotations

import ctypes

import numpy as np

import qne as Q

_hip = None
H2D, D2H, D2D = 1, 2, 3


def hip():
    global _hip
    if _hip is None:
        Q.load_library()  # binds libamdhip64.so.7; the name below resolves to that same object
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        h.hipFree.argtypes = [ctypes.c_void_p]
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
        h.hipGetErrorString.argtypes = [ctypes.c_int]
        h.hipGetErrorString.restype = ctypes.c_char_p
        vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        h.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
        h.hipStreamCreate.argtypes = [pvp]
        h.hipStreamDestroy.argtypes = [vp]
        h.hipStreamSynchronize.argtypes = [vp]
        h.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [vp, pvp]
        h.hipGraphInstantiate.argtypes = [pvp, vp, vp, vp, ctypes.c_size_t]
        h.hipGraphLaunch.argtypes = [vp, vp]
        h.hipGraphExecDestroy.argtypes = [vp]
        h.hipGraphDestroy.argtypes = [vp]
        for f in (h.hipMalloc, h.hipFree, h.hipMemcpy, h.hipMemset, h.hipDeviceSynchronize, h.hipMemGetInfo,
                  h.hipStreamCreate, h.hipStreamDestroy, h.hipStreamSynchronize, h.hipStreamBeginCapture,
                  h.hipStreamEndCapture, h.hipGraphInstantiate, h.hipGraphLaunch, h.hipGraphExecDestroy,
                  h.hipGraphDestroy):
            f.restype = ctypes.c_int
        _hip = h
    return _hip


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(rc).decode()}")


class DeviceArray:
    """A device allocation with a numpy shape and dtype."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 16)), "hipMalloc")
        self.ptr = p.value

    def data_ptr(self) -> int:
        return self.ptr

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        check(hip().hipMemcpy(self.ptr, a.ctypes.data, self.nbytes, H2D), "hipMemcpy H2D")
        return self

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        check(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")
        return self

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def to_dev(a) -> DeviceArray:
    a = np.ascontiguousarray(a)
    return DeviceArray(a.shape, a.dtype).upload(a)


def empty(shape, dtype=np.float32) -> DeviceArray:
    return DeviceArray(shape, dtype)


def empty_like(d: DeviceArray) -> DeviceArray:
    return DeviceArray(d.shape, d.dtype)


def zeros(shape, dtype=np.float32) -> DeviceArray:
    return DeviceArray(shape, dtype).zero()


def sync():
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_free() -> int:
    """Free device memory in bytes (hipMemGetInfo)."""
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    check(hip().hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)), "hipMemGetInfo")
    return int(free.value)


class Stream:
    """A created HIP stream (default priority), with graph capture of the work enqueued on it."""

    CAPTURE_GLOBAL = 0  # hipStreamCaptureModeGlobal

    def __init__(self):
        p = ctypes.c_void_p()
        check(hip().hipStreamCreate(ctypes.byref(p)), "hipStreamCreate")
        self.ptr = p.value

    def sync(self):
        check(hip().hipStreamSynchronize(self.ptr), "hipStreamSynchronize")

    def capture(self, enqueue):
        """Captures what enqueue() puts on this stream; returns an instantiated graph."""
        check(hip().hipStreamBeginCapture(self.ptr, self.CAPTURE_GLOBAL), "hipStreamBeginCapture")
        g = ctypes.c_void_p()
        try:
            enqueue()
        finally:
            rc = hip().hipStreamEndCapture(self.ptr, ctypes.byref(g))
        check(rc, "hipStreamEndCapture")
        e = ctypes.c_void_p()
        try:
            check(hip().hipGraphInstantiate(ctypes.byref(e), g, None, None, 0), "hipGraphInstantiate")
        finally:
            hip().hipGraphDestroy(g)
        return Graph(e.value)

    def destroy(self):
        if self.ptr:
            hip().hipStreamDestroy(self.ptr)
            self.ptr = 0


class Graph:
    def __init__(self, exec_ptr):
        self.ptr = exec_ptr

    def launch(self, stream: Stream):
        check(hip().hipGraphLaunch(self.ptr, stream.ptr), "hipGraphLaunch")

    def destroy(self):
        if self.ptr:
            hip().hipGraphExecDestroy(self.ptr)
            self.ptr = 0


def mapped_hip_runtimes() -> list[str]:
    """Paths of every HIP / HSA runtime library mapped into this process."""
    seen = []
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and ("libamdhip64" in parts[-1] or "libhsa-runtime64" in parts[-1]):
                if parts[-1] not in seen:
                    seen.append(parts[-1])
    return seen
