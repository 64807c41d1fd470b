"""Device buffers for tests that call the device-pointer entry points:
hipMalloc / hipMemcpy / hipFree through the HIP runtime the backend library
itself links (one runtime per process).  Test infrastructure only."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_hip = None


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        import talos_amd
        talos_amd.lib()  # loads the backend, and with it its HIP runtime
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        _hip = C.CDLL(path or os.path.join("/opt/rocm/lib", "libamdhip64.so"))
        _hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        _hip.hipFree.argtypes = [C.c_void_p]
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipDeviceSynchronize.argtypes = []
    return _hip


class DeviceBuffer:
    """nbytes of device memory; upload / download numpy arrays."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        rc = hip().hipMalloc(C.byref(p), nbytes)
        if rc != 0:
            raise RuntimeError(f"hipMalloc({nbytes}) failed: {rc}")
        self.ptr = p.value
        self.nbytes = nbytes

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        assert hip().hipMemcpy(C.c_void_p(self.ptr), C.c_void_p(a.ctypes.data), a.nbytes, 1) == 0

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        assert hip().hipMemcpy(C.c_void_p(out.ctypes.data), C.c_void_p(self.ptr), out.nbytes, 2) == 0
        return out

    def free(self):
        if self.ptr:
            hip().hipFree(C.c_void_p(self.ptr))
            self.ptr = None
