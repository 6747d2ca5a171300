"""Device-buffer helpers for the GPU tests (through the C ABI only)."""
import ctypes as C

import numpy as np

from atlas_amd._lib import check, check_void, load
from atlas_amd.tensor import GpuBuf, _DevMem


class Dev:
    """A device copy of a numpy array (any dtype)."""

    def __init__(self, a: np.ndarray):
        self.a = np.ascontiguousarray(a)
        self.mem = _DevMem(max(self.a.nbytes, 4), sync_alloc=True)
        if self.a.nbytes:
            check(load().atlas_memcpy_h2d(self.mem.ptr, self.a.ctypes.data_as(C.c_void_p),
                                          self.a.nbytes))

    @staticmethod
    def empty(shape, dtype=np.float32):
        return Dev(np.zeros(shape, dtype))

    @property
    def ptr(self):
        return self.mem.ptr

    def get(self) -> np.ndarray:
        out = np.empty_like(self.a)
        check(load().atlas_memcpy_d2h(out.ctypes.data_as(C.c_void_p), self.mem.ptr, out.nbytes))
        return out


def lib():
    return load()


def sync():
    load().atlas_sync()
    check_void()


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))
