"""Device buffers for device-resident inputs (an encoder output that already lives on the GPU), made
through the same HIP runtime libw4h.so is linked against, over ctypes.

torch is not used for this: its ROCm wheel carries its own HIP runtime, and a process that has
loaded libw4h.so (and with it the system runtime) cannot bring torch's runtime up on the same GPU.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

_HIP = None
_H2D, _D2H = 1, 2


def _hip():
    global _HIP
    if _HIP is None:
        _lib.lib()  # the library first, so the runtime below is the one it already loaded
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        h.hipFree.argtypes = [ctypes.c_void_p]
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipSetDevice.argtypes = [ctypes.c_int]
        _HIP = h
    return _HIP


class DeviceArray:
    """A device copy of a host array on `device` (freed by close() or on leaving a with block)."""

    def __init__(self, a: np.ndarray, device: int = 0):
        a = np.ascontiguousarray(a)
        self.shape, self.dtype, self.nbytes = a.shape, a.dtype, a.nbytes
        self._ptr = ctypes.c_void_p()
        h = _hip()
        if h.hipSetDevice(device) != 0:
            raise RuntimeError(f"hipSetDevice({device}) failed")
        if h.hipMalloc(ctypes.byref(self._ptr), max(a.nbytes, 1)) != 0:
            raise RuntimeError(f"hipMalloc of {a.nbytes} bytes failed")
        if h.hipMemcpy(self._ptr, a.ctypes.data, a.nbytes, _H2D) != 0:
            self.close()
            raise RuntimeError("hipMemcpy host to device failed")

    @property
    def address(self) -> int:
        if not self._ptr.value:
            raise ValueError("closed DeviceArray")
        return self._ptr.value

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if _hip().hipMemcpy(out.ctypes.data, self._ptr, self.nbytes, _D2H) != 0:
            raise RuntimeError("hipMemcpy device to host failed")
        return out

    def close(self) -> None:
        if self._ptr.value:
            _hip().hipFree(self._ptr)
            self._ptr = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
