"""Minimal HIP runtime plumbing over ctypes: device<->host copies of raw
pointers (the layer arena, expert matrices). Used by tests and the benchmark."""
import ctypes

import numpy as np

_hip = None


def hip():
    global _hip
    if _hip is None:
        from hy3_amd import one_hip_runtime
        one_hip_runtime()
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipDeviceSynchronize.restype = ctypes.c_int
    return _hip


def to_host(dev_ptr, nbytes, dtype=np.uint8):
    out = np.empty(nbytes, np.uint8)
    rc = hip().hipMemcpy(out.ctypes.data, dev_ptr, nbytes, 2)  # hipMemcpyDeviceToHost
    if rc != 0:
        raise RuntimeError(f"hipMemcpy D2H failed: {rc}")
    return out.view(dtype)


def to_device(dev_ptr, arr):
    arr = np.ascontiguousarray(arr)
    rc = hip().hipMemcpy(dev_ptr, arr.ctypes.data, arr.nbytes, 1)  # hipMemcpyHostToDevice
    if rc != 0:
        raise RuntimeError(f"hipMemcpy H2D failed: {rc}")
