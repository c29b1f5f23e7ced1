"""Pinned, device-mapped, coherent host buffers (mailbox words, host-published x rows and picks, host partials,
host-resident expert copies), allocated through the C ABI and exposed as numpy arrays."""
import ctypes

import numpy as np

from . import _lib


class HostBuffer:
    """A host allocation visible to the GPU at the same address (coherent: GPU writes followed by a system
    fence are visible to the CPU, and CPU writes to the GPU)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _lib.call("mm_host_alloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = p.value
        self._raw = (ctypes.c_uint8 * max(self.nbytes, 1)).from_address(self.ptr)

    def array(self, dtype, shape=None, offset=0):
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if shape is None else int(np.prod(shape))
        a = np.frombuffer(self._raw, dtype=dt, count=n, offset=offset)
        return a if shape is None else a.reshape(shape)

    def data_ptr(self, offset=0):
        return self.ptr + offset

    def free(self):
        if self.ptr:
            _lib.call("mm_host_free", self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
