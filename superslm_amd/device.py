"""Device buffers through libsslm_hip.so's own HIP runtime.

The backend links ROCm's HIP runtime; a second HIP runtime in the same process (for example the
one bundled with PyTorch) would not see the device once this one owns it, so host code that
drives the backend allocates and copies through these helpers instead."""
from __future__ import annotations

import ctypes

import numpy as np


class Device:
    def __init__(self, lib):
        self.lib = lib
        L = lib.lib
        L.sslm_hip_device_alloc.restype = ctypes.c_void_p
        L.sslm_hip_device_alloc.argtypes = [ctypes.c_size_t]
        L.sslm_hip_device_free.argtypes = [ctypes.c_void_p]
        L.sslm_hip_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        L.sslm_hip_synchronize.argtypes = []

    def upload(self, arr: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(arr)
        d = DeviceArray(self, a.shape, a.dtype)
        self.lib.check("copy h2d", self.lib.lib.sslm_hip_copy(d.ptr, a.ctypes.data, a.nbytes, 0))
        return d

    def zeros(self, shape, dtype) -> "DeviceArray":
        return self.upload(np.zeros(shape, dtype=dtype))

    def copy_device(self, dst: "DeviceArray", src: "DeviceArray"):
        n = min(dst.nbytes, src.nbytes)
        self.lib.check("copy d2d", self.lib.lib.sslm_hip_copy(dst.ptr, src.ptr, n, 2))


class DeviceArray:
    def __init__(self, dev: Device, shape, dtype):
        self.dev = dev
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = dev.lib.lib.sslm_hip_device_alloc(max(1, self.nbytes))
        if not self.ptr:
            raise MemoryError("device allocation failed")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        self.dev.lib.check("copy d2h", self.dev.lib.lib.sslm_hip_copy(out.ctypes.data, self.ptr, self.nbytes, 1))
        return out

    def free(self):
        if self.ptr:
            self.dev.lib.lib.sslm_hip_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
