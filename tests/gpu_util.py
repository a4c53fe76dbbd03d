"""Device-buffer plumbing for the GPU tests.  Memory comes from the engine's
own C ABI (gsdh_malloc / gsdh_memcpy_*): torch ships a second HIP runtime
(its bundled libamdhip64) that must not share a process with the engine's."""
import ctypes

import numpy as np


class DBuf:
    """A device allocation of the engine library; freed with the object."""

    def __init__(self, nbytes: int):
        from gsdlq import hip
        self._lib = hip.lib()
        self.nbytes = max(int(nbytes), 16)
        self.ptr = ctypes.c_void_p()
        self._lib.gsdh_malloc(ctypes.byref(self.ptr), self.nbytes)
        zeros = np.zeros(self.nbytes, np.uint8)
        self._lib.gsdh_memcpy_h2d(self.ptr, zeros.ctypes.data_as(ctypes.c_void_p), self.nbytes, None)
        self._lib.gsdh_stream_sync(None)

    def __del__(self):
        try:
            if self.ptr:
                self._lib.gsdh_free(self.ptr)
                self.ptr = None
        except Exception:
            pass


def D(a):
    """Copy a numpy array's bytes into a new device buffer."""
    a = np.ascontiguousarray(a)
    b = DBuf(a.nbytes)
    if a.nbytes:
        b._lib.gsdh_memcpy_h2d(b.ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, None)
        b._lib.gsdh_stream_sync(None)
    return b


def E(nbytes):
    return DBuf(nbytes)


def H(b, dtype, count=None):
    """Synchronise and copy a device buffer back as a numpy array."""
    b._lib.gsdh_stream_sync(None)
    out = np.empty(b.nbytes, np.uint8)
    b._lib.gsdh_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), b.ptr, b.nbytes, None)
    b._lib.gsdh_stream_sync(None)
    a = out[: (b.nbytes // np.dtype(dtype).itemsize) * np.dtype(dtype).itemsize].view(dtype)
    return a if count is None else a[:count].copy()


def p(b):
    return None if b is None else b.ptr


def banner(msg):
    print(f"\n[gpu-test] {msg}", flush=True)
