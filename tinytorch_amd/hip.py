"""Device buffers and stream timing through the library's own C ABI.

PyTorch is deliberately not used here: its wheel bundles a second copy of the
HIP runtime, and two HIP runtimes in one process do not share devices,
pointers or streams.  Everything goes through build/libtinytorch.so.
"""
import ctypes

import numpy as np

from . import lib


class DevBuf:
    """A device allocation of `n` float32 (or int32) elements."""

    def __init__(self, n, dtype=np.float32):
        self.dtype = np.dtype(dtype)
        self.n = int(n)
        self.nbytes = max(self.n, 1) * self.dtype.itemsize
        self.ptr = lib().tth_malloc(self.nbytes)
        if not self.ptr:
            raise MemoryError(f"tth_malloc({self.nbytes}) failed (error {lib().tth_last_error()})")

    @classmethod
    def from_np(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.size, arr.dtype)
        if arr.size and lib().tth_h2d(b.ptr, arr.ctypes.data, arr.nbytes) != 0:
            raise RuntimeError("tth_h2d failed")
        return b

    def to_np(self, shape=None):
        out = np.empty(self.n, dtype=self.dtype)
        if self.n and lib().tth_d2h(out.ctypes.data, self.ptr, out.nbytes) != 0:
            raise RuntimeError("tth_d2h failed")
        return out.reshape(shape) if shape is not None else out

    def fill(self, v):
        check(lib().tt_k_fill(self.ptr, self.n, ctypes.c_float(v)), "tt_k_fill")

    def free(self):
        if self.ptr:
            lib().tth_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed with {rc} (runtime error {lib().tth_last_error()})")


def sync():
    check(lib().tth_sync(), "tth_sync")


class StreamTimer:
    """Times enqueued work with two HIP events on the library stream."""

    def __init__(self):
        self.a = lib().tth_event_create()
        self.b = lib().tth_event_create()
        if not self.a or not self.b:
            raise RuntimeError("tth_event_create failed")

    def start(self):
        check(lib().tth_event_record(self.a), "tth_event_record")

    def stop_ms(self):
        check(lib().tth_event_record(self.b), "tth_event_record")
        ms = lib().tth_event_elapsed_ms(self.a, self.b)
        if ms < 0:
            raise RuntimeError("tth_event_elapsed_ms failed")
        return float(ms)

    def __del__(self):
        try:
            lib().tth_event_destroy(self.a)
            lib().tth_event_destroy(self.b)
        except Exception:
            pass
