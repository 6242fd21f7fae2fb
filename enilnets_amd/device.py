"""Device memory owned by libenilnets_amd.

``DeviceArray`` is a dense, row-major array in HBM with a NumPy dtype and
shape.  It is what the device-resident API (``enilnets_amd.nn``) and
the benchmark keep between calls; the NumPy drop-in functions create and
release them per call.
"""

import ctypes
import math
from typing import Sequence, Tuple

import numpy as np

from . import _lib


class DeviceArray:
    """A dense row-major device array."""

    __slots__ = ("shape", "dtype", "_ptr", "nbytes", "_owner", "__weakref__")

    def __init__(self, shape: Sequence[int], dtype, ptr: int = None, owner=None):
        self.shape: Tuple[int, ...] = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = math.prod(self.shape) * self.dtype.itemsize
        self._owner = owner
        if ptr is None:
            p = ctypes.c_void_p()
            _lib.call("enq_malloc", ctypes.byref(p), ctypes.c_size_t(self.nbytes))
            self._ptr = p.value or 0
        else:
            self._ptr = int(ptr)

    # -- construction -----------------------------------------------------
    @classmethod
    def empty(cls, shape, dtype) -> "DeviceArray":
        return cls(shape, dtype)

    @classmethod
    def from_numpy(cls, arr) -> "DeviceArray":
        a = np.ascontiguousarray(arr)
        out = cls(a.shape, a.dtype)
        if a.nbytes:
            _lib.call("enq_copy_to_device", out.ptr, a.ctypes.data_as(ctypes.c_void_p),
                      ctypes.c_size_t(a.nbytes))
        return out

    # -- access -----------------------------------------------------------
    @property
    def ptr(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(self._ptr)

    @property
    def address(self) -> int:
        return self._ptr

    @property
    def size(self) -> int:
        return math.prod(self.shape)

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def numpy(self) -> np.ndarray:
        """Copy to a new host array (waits for pending work on the stream)."""
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            _lib.call("enq_copy_to_host", out.ctypes.data_as(ctypes.c_void_p), self.ptr,
                      ctypes.c_size_t(self.nbytes))
        return out

    def copy_from(self, arr) -> None:
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        if a.shape != self.shape:
            raise ValueError(f"shape {a.shape} does not match device array {self.shape}")
        if a.nbytes:
            _lib.call("enq_copy_to_device", self.ptr, a.ctypes.data_as(ctypes.c_void_p),
                      ctypes.c_size_t(a.nbytes))

    def reshape(self, *shape) -> "DeviceArray":
        """A view with another shape over the same memory."""
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(shape)
        if -1 in shape:
            i = shape.index(-1)
            rest = int(np.prod([s for j, s in enumerate(shape) if j != i], dtype=np.int64))
            shape[i] = self.size // max(rest, 1)
        if int(np.prod(shape, dtype=np.int64)) != self.size:
            raise ValueError(f"cannot reshape {self.shape} to {tuple(shape)}")
        return DeviceArray(shape, self.dtype, ptr=self._ptr, owner=self)

    def free(self) -> None:
        if self._owner is None and self._ptr:
            _lib.call("enq_free", ctypes.c_void_p(self._ptr))
        self._ptr = 0

    def __del__(self):
        try:
            if self._owner is None and self._ptr and _lib._lib is not None:
                _lib._lib.enq_free(ctypes.c_void_p(self._ptr))
                self._ptr = 0
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}, ptr=0x{self._ptr:x})"

    def __deepcopy__(self, memo):
        out = DeviceArray(self.shape, self.dtype)
        if self.nbytes:
            _lib.call("enq_copy_on_device", out.ptr, self.ptr, ctypes.c_size_t(self.nbytes))
        return out


def null() -> ctypes.c_void_p:
    return ctypes.c_void_p(0)
