"""ctypes Tensor / Node wrapper over the GPU backend.

Same classes, methods and error behaviour as the reference's ctypes wrapper
(reference tests/torch_py.py:80-203): a NULL from the C layer raises
ValueError, a backward seed of the wrong length raises ValueError before the
C call, seeds of any dtype/contiguity are coerced to contiguous float32.
The library is loaded from build/ (built by `make lib`); it is never built
here.
"""
import ctypes

import numpy as np

from . import F32P, lib

LIB = lib()


def _checked(ptr, op):
    if not ptr:
        raise ValueError(f"tinytorch: {op} failed (invalid arguments or shape mismatch)")
    return ptr


class Tensor:
    """Owns a C Tensor reference; release() or GC drops it."""

    def __init__(self, ptr, owned=True):
        self.ptr = ptr
        self.owned = owned

    @classmethod
    def from_np(cls, arr):
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        shape = (ctypes.c_long * max(arr.ndim, 1))(*arr.shape)
        return cls(_checked(LIB.tt_fromdata(arr.ctypes.data_as(F32P), shape, arr.ndim),
                            "tt_fromdata"))

    def shape(self):
        nd = int(LIB.tt_ndim(self.ptr))
        shp = (ctypes.c_long * max(nd, 1))()
        LIB.tt_shape(self.ptr, shp)
        return tuple(shp)[:nd]

    def to_np(self):
        n = int(LIB.tt_numel(self.ptr))
        data = LIB.tt_data(self.ptr)
        if not data:
            raise RuntimeError("tinytorch: device to host copy failed")
        buf = np.ctypeslib.as_array(data, shape=(max(n, 1),))
        return buf[:n].copy().reshape(self.shape())

    def release(self):
        if self.ptr and self.owned:
            LIB.tt_release(self.ptr)
        self.ptr = None


class Node:
    """Owns an AGNode reference; call release() when done."""

    def __init__(self, ptr):
        self.ptr = ptr

    @classmethod
    def leaf(cls, arr, requires_grad=True):
        t = Tensor.from_np(arr)
        n = cls(_checked(LIB.ag_leaf(t.ptr, 1 if requires_grad else 0), "ag_leaf"))
        t.release()  # the node holds its own reference
        return n

    def detach(self, requires_grad=True):
        """A new leaf sharing this node's value tensor (no copy, fresh grad):
        how device-resident parameters are re-entered into each step's graph."""
        return Node(_checked(LIB.ag_leaf(LIB.ag_value(self.ptr), 1 if requires_grad else 0),
                             "ag_leaf"))

    def value(self):
        return Tensor(LIB.ag_value(self.ptr), owned=False).to_np()

    def grad(self):
        g = LIB.ag_grad(self.ptr)
        return None if not g else Tensor(g, owned=False).to_np()

    def backward(self, seed=None):
        if seed is None:
            LIB.ag_backward(self.ptr)
            return
        seed = np.ascontiguousarray(seed, dtype=np.float32)
        need = int(LIB.tt_numel(LIB.ag_value(self.ptr)))
        if int(seed.size) != need:
            raise ValueError(f"tinytorch: seed length mismatch (got {int(seed.size)}, need {need})")
        LIB.ag_backward_from(self.ptr, seed.ctypes.data_as(F32P), int(seed.size))

    def __add__(self, other):
        if isinstance(other, (int, float)):
            return Node(_checked(LIB.ag_addscalar(self.ptr, ctypes.c_float(other)), "ag_addscalar"))
        return Node(_checked(LIB.ag_add(self.ptr, other.ptr), "ag_add"))

    def __mul__(self, other):
        if isinstance(other, (int, float)):
            return Node(_checked(LIB.ag_mulscalar(self.ptr, ctypes.c_float(other)), "ag_mulscalar"))
        return Node(_checked(LIB.ag_mul(self.ptr, other.ptr), "ag_mul"))

    def __rmul__(self, other):
        return self.__mul__(other)

    def matmul(self, other):
        return Node(_checked(LIB.ag_matmul(self.ptr, other.ptr), "ag_matmul"))

    def relu(self):
        return Node(_checked(LIB.ag_relu(self.ptr), "ag_relu"))

    def softmax(self):
        return Node(_checked(LIB.ag_softmax(self.ptr), "ag_softmax"))

    def padones(self):
        return Node(_checked(LIB.ag_padones(self.ptr), "ag_padones"))

    def reshape(self, shape):
        c_shape = (ctypes.c_long * len(shape))(*shape)
        return Node(_checked(LIB.ag_reshape(self.ptr, c_shape, len(shape)), "ag_reshape"))

    def conv2d(self, w, b=None, stride=1, pad=0):
        sh, sw = (stride, stride) if isinstance(stride, int) else stride
        ph, pw = (pad, pad) if isinstance(pad, int) else pad
        return Node(_checked(LIB.ag_conv2d(self.ptr, w.ptr, b.ptr if b else None, sh, sw, ph, pw),
                             "ag_conv2d"))

    def maxpool2d(self, pool_size=2, stride=2):
        ph, pw = (pool_size, pool_size) if isinstance(pool_size, int) else pool_size
        sh, sw = (stride, stride) if isinstance(stride, int) else stride
        return Node(_checked(LIB.ag_maxpool2d(self.ptr, ph, pw, sh, sw), "ag_maxpool2d"))

    def avgpool2d(self, pool_size=2, stride=2):
        ph, pw = (pool_size, pool_size) if isinstance(pool_size, int) else pool_size
        sh, sw = (stride, stride) if isinstance(stride, int) else stride
        return Node(_checked(LIB.ag_avgpool2d(self.ptr, ph, pw, sh, sw), "ag_avgpool2d"))

    # ---- additions of this backend ----
    def softmax_ce(self, labels):
        lab = np.ascontiguousarray(labels, dtype=np.int32)
        return Node(_checked(LIB.ag_softmax_ce(self.ptr, lab.ctypes.data_as(
            ctypes.POINTER(ctypes.c_int)), lab.size), "ag_softmax_ce"))

    def probs(self):
        p = LIB.ag_softmax_ce_probs(self.ptr)
        return None if not p else Tensor(p, owned=False).to_np()

    def sgd_step(self, lr):
        if LIB.ag_sgd_step(self.ptr, ctypes.c_float(lr)) != 0:
            raise RuntimeError("tinytorch: sgd step failed")

    def release(self):
        if self.ptr:
            LIB.ag_release(self.ptr)
            self.ptr = None


class Optim:
    """Optimizer with device-resident state (SGD-momentum or Adam).

    The update rules are the reference harness's NumPy optimizers
    (reference tests/gate_mnist_mlp.py:121-124, tests/gate_cifar_cnn.py:81-98)
    run on the GPU; step(params) takes the parameter nodes in the same order
    on every call."""

    def __init__(self, ptr):
        if not ptr:
            raise ValueError("tinytorch: invalid optimizer arguments")
        self.ptr = ptr

    @classmethod
    def sgd_momentum(cls, lr, momentum):
        return cls(LIB.ag_optim_sgd_momentum(lr, momentum))

    @classmethod
    def adam(cls, lr=0.003, beta1=0.9, beta2=0.999, eps=1e-8):
        return cls(LIB.ag_optim_adam(lr, beta1, beta2, eps))

    def step(self, params):
        arr = (ctypes.c_void_p * len(params))(*[p.ptr for p in params])
        if LIB.ag_optim_step(self.ptr, arr, len(params)) != 0:
            raise ValueError("tinytorch: optimizer step failed (parameter list or sizes changed?)")

    @property
    def t(self):
        return LIB.ag_optim_steps(self.ptr)

    @property
    def lr(self):
        return LIB.ag_optim_lr(self.ptr)

    @lr.setter
    def lr(self, value):
        LIB.ag_optim_set_lr(self.ptr, float(value))

    def release(self):
        if self.ptr:
            LIB.ag_optim_release(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

