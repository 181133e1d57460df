"""Minimal HIP runtime access through ctypes for the GPU tests (device
buffers of numpy arrays)."""

import ctypes

import numpy as np

_hip = None


def hip():
    global _hip
    if _hip is None:
        h = ctypes.CDLL("libamdhip64.so")
        h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipFree.argtypes = [ctypes.c_void_p]
        h.hipDeviceSynchronize.argtypes = []
        _hip = h
    return _hip


class DeviceArray:
    """A device copy of a numpy array (freed with the object)."""

    def __init__(self, a):
        self.a = np.ascontiguousarray(a)
        self.ptr = ctypes.c_void_p()
        n = max(self.a.nbytes, 4)
        if hip().hipMalloc(ctypes.byref(self.ptr), ctypes.c_size_t(n)) != 0:
            raise MemoryError("hipMalloc failed")
        if self.a.nbytes and hip().hipMemcpy(self.ptr, self.a.ctypes.data_as(ctypes.c_void_p),
                                             ctypes.c_size_t(self.a.nbytes), 1) != 0:
            raise RuntimeError("hipMemcpy to device failed")

    @property
    def value(self):
        return self.ptr.value

    def get(self):
        out = np.empty_like(self.a)
        if out.nbytes and hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr,
                                          ctypes.c_size_t(out.nbytes), 2) != 0:
            raise RuntimeError("hipMemcpy to host failed")
        return out

    def __del__(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()
