"""Device-resident datasets (ctypes side of include/tt_data.h).

Replaces the reference harnesses' NumPy data path -- read the files,
normalise on the host, copy every minibatch (reference
tests/gate_mnist_mlp.py:37-53,83-87, tests/gate_cifar_cnn.py:47-68,165) --
with one upload of the uint8 samples and a gather+normalise kernel per
batch.  Files are read from local paths only."""
import ctypes

import numpy as np

from . import F32P, lib
from .torch_py import Node, _checked

LIB = lib()

MNIST_MEAN, MNIST_STD = (0.1307,), (0.3081,)          # tests/gate_mnist_mlp.py:84
CIFAR_MEAN = (0.4914, 0.4822, 0.4465)                 # tests/gate_cifar_cnn.py:132-133
CIFAR_STD = (0.2023, 0.1994, 0.2010)


def idx_probe(path):
    """(dims) of a uint8 idx file, read from its header (no GPU needed)."""
    nd = ctypes.c_int()
    dims = (ctypes.c_long * 8)()
    if LIB.tt_idx_probe(path.encode(), ctypes.byref(nd), dims) != 0:
        raise ValueError(f"tinytorch: {path} is not a uint8 idx file")
    return tuple(dims[: nd.value])


class Dataset:
    """uint8 samples in HBM; batch(idx) returns a normalised float32 leaf."""

    def __init__(self, ptr, mean, std):
        self.ptr = _checked(ptr, "dataset load")
        c, h, w = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        LIB.tt_dataset_shape(self.ptr, ctypes.byref(c), ctypes.byref(h), ctypes.byref(w))
        self.shape = (c.value, h.value, w.value)
        self.mean = np.ascontiguousarray(mean, np.float32)
        self.std = np.ascontiguousarray(std, np.float32)
        if self.mean.size != c.value or self.std.size != c.value:
            raise ValueError("tinytorch: mean/std need one value per channel")

    @classmethod
    def mnist(cls, images_path, labels_path, mean=MNIST_MEAN, std=MNIST_STD):
        return cls(LIB.tt_dataset_idx(images_path.encode(), labels_path.encode()), mean, std)

    @classmethod
    def cifar10(cls, paths, mean=CIFAR_MEAN, std=CIFAR_STD):
        arr = (ctypes.c_char_p * len(paths))(*[p.encode() for p in paths])
        return cls(LIB.tt_dataset_cifar10_bin(arr, len(paths)), mean, std)

    @classmethod
    def from_u8(cls, samples, labels, mean, std):
        s = np.ascontiguousarray(samples, np.uint8)
        lab = np.ascontiguousarray(labels, np.int32)
        n, c, h, w = s.shape
        return cls(LIB.tt_dataset_from_u8(s.ctypes.data, lab.ctypes.data, n, c, h, w), mean, std)

    def __len__(self):
        return int(LIB.tt_dataset_len(self.ptr))

    def labels(self):
        out = np.empty(len(self), np.int32)
        LIB.tt_dataset_labels(self.ptr, out.ctypes.data)
        return out

    def batch(self, idx, flat=False, requires_grad=False):
        """(leaf node of shape (n, c, h, w) or (n, c*h*w), int32 labels)"""
        idx = np.ascontiguousarray(idx, np.int64)
        lab = np.empty(idx.size, np.int32)
        t = _checked(LIB.tt_dataset_batch(self.ptr, idx.ctypes.data, idx.size,
                                          self.mean.ctypes.data_as(F32P),
                                          self.std.ctypes.data_as(F32P), 1 if flat else 0,
                                          lab.ctypes.data), "tt_dataset_batch")
        n = Node(_checked(LIB.ag_leaf(t, 1 if requires_grad else 0), "ag_leaf"))
        LIB.tt_release(t)
        return n, lab

    def release(self):
        if self.ptr:
            LIB.tt_dataset_release(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass
