"""Device buffers for the tests of entry points that take device pointers."""

import ctypes as C

import numpy as np


class Device:
    """Device buffers through the HIP runtime (the library takes device pointers)."""

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        for name in ("hipMalloc", "hipFree", "hipMemcpy", "hipDeviceSynchronize"):
            getattr(self.L, name).restype = C.c_int
        self.held = []

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        p = C.c_void_p()
        assert self.L.hipMalloc(C.byref(p), C.c_size_t(arr.nbytes)) == 0
        self.held.append(p)
        assert self.L.hipMemcpy(p, arr.ctypes.data_as(C.c_void_p), C.c_size_t(arr.nbytes), 1) == 0
        return p

    def empty(self, nbytes):
        p = C.c_void_p()
        assert self.L.hipMalloc(C.byref(p), C.c_size_t(nbytes)) == 0
        self.held.append(p)
        return p

    def download(self, p, shape):
        out = np.empty(shape, np.float32)
        assert self.L.hipDeviceSynchronize() == 0
        assert self.L.hipMemcpy(out.ctypes.data_as(C.c_void_p), p, C.c_size_t(out.nbytes), 2) == 0
        return out

    def free(self):
        self.L.hipDeviceSynchronize()
        for p in self.held:
            self.L.hipFree(p)
        self.held = []
