"""Pinned, device-mapped, coherent host buffers (mailbox words, host-published x rows and picks, host partials,
host-resident expert copies), allocated through the C ABI and exposed as numpy arrays."""
import ctypes

import numpy as np

from . import _lib


class HostBuffer:
    """A host allocation visible to the GPU at the same address (coherent: GPU writes followed by a system
    fence are visible to the CPU, and CPU writes to the GPU)."""

    def __init__(self, nbytes):
        self.holders = 0          # users that read the memory from other threads (the host tier): free() refuses
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

    def hold(self):
        """Mark the memory as read by a thread this object does not control (the host tier's workers); free() is
        refused until release(). The holder keeps a reference, so garbage collection cannot free it either."""
        self.holders += 1

    def release(self):
        self.holders = max(0, self.holders - 1)

    def free(self):
        if self.holders:
            raise RuntimeError("HostBuffer.free: the memory is still read by the host tier (shut it down first)")
        if self.ptr:
            _lib.call("mm_host_free", self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
