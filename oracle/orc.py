"""ORACLE -- test infrastructure only.

ctypes wrappers over oracle/build/liborc.so (the C restatement of the
reference CPU path, oracle/orc.c) and, when it has been built, over
oracle/_ref/libtinytorch_ref.so (the reference's own C sources compiled by
oracle/Makefile).  Imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg; never by the product package.
"""
import ctypes
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORC_PATH = os.path.join(HERE, "build", "liborc.so")
REF_PATH = os.path.join(HERE, "_ref", "libtinytorch_ref.so")

_I, _L, _F, _D, _V = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_double, ctypes.c_void_p
_ORC = None
_REF = None


def _p(a):
    return None if a is None else a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def orc():
    global _ORC
    if _ORC is None:
        if not os.path.exists(ORC_PATH):
            raise RuntimeError(f"{ORC_PATH} not built (make -C oracle)")
        h = ctypes.CDLL(ORC_PATH)
        sig = {
            "orc_sgemm": (_I, [_I, _I, _I, _V, _V, _V, _I]),
            "orc_matmul_naive": (None, [_I, _I, _I, _V, _V, _V]),
            "orc_matmul_nt": (None, [_I, _I, _I, _V, _V, _V]),
            "orc_matmul_tn": (None, [_I, _I, _I, _V, _V, _V]),
            "orc_sgemm_a_bt": (None, [_I, _I, _L, _V, _V, _V]),
            "orc_im2col": (None, [_V] + [_I] * 10 + [_V]),
            "orc_col2im": (None, [_V] + [_I] * 10 + [_V]),
            "orc_conv2d_fwd": (_I, [_V, _I, _I, _I, _I, _V, _I, _I, _I, _V, _I, _I, _I, _I, _V, _I]),
            "orc_conv2d_bwd": (_I, [_V, _I, _I, _I, _I, _V, _I, _I, _I, _V, _I, _I, _I, _I,
                                    _V, _V, _V, _I]),
            "orc_bias_grad": (None, [_V, _I, _I, _I, _V]),
            "orc_maxpool_fwd": (None, [_V] + [_I] * 8 + [_V]),
            "orc_maxpool_bwd": (None, [_V, _V] + [_I] * 8 + [_V]),
            "orc_avgpool_fwd": (None, [_V] + [_I] * 8 + [_V]),
            "orc_avgpool_bwd": (None, [_V] + [_I] * 8 + [_V]),
            "orc_relu_fwd": (None, [_V, _V, _L]),
            "orc_relu_bwd": (None, [_V, _V, _V, _L]),
            "orc_softmax_fwd": (None, [_V, _V, _L, _I]),
            "orc_softmax_bwd": (None, [_V, _V, _V, _L, _I]),
            "orc_padones_fwd": (None, [_V, _V, _L, _L]),
            "orc_padones_bwd": (None, [_V, _V, _L, _L]),
            "orc_ce_seed": (_D, [_V, _V, _L, _I, _V]),
            "orc_mlp_step": (_D, [_I] * 5 + [_V] * 10 + [_I]),
            "orc_cnn_step": (_D, [_I] * 7 + [_V] * 14 + [_I]),
            "orc_fill_uniform": (None, [_V, _L, _F, _F, ctypes.c_ulonglong]),
            "orc_fill_normal": (None, [_V, _L, _F, ctypes.c_ulonglong]),
            "orc_fill_labels": (None, [_V, _L, _I, ctypes.c_ulonglong]),
        }
        for name, (res, args) in sig.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _ORC = h
    return _ORC


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    """The reference library built from its own sources (tensor.h/autograd.h ABI)."""
    global _REF
    if _REF is None:
        if not ref_available():
            raise RuntimeError(f"{REF_PATH} not built (make -C oracle ref)")
        h = ctypes.CDLL(REF_PATH)
        F32P = ctypes.POINTER(ctypes.c_float)
        I64P = ctypes.POINTER(ctypes.c_long)
        sig = {
            "tt_new": (_V, [I64P, _I]), "tt_fromdata": (_V, [F32P, I64P, _I]),
            "tt_release": (None, [_V]), "tt_data": (F32P, [_V]), "tt_numel": (_L, [_V]),
            "tt_matmul": (_V, [_V, _V]), "tt_matmul_omp": (_V, [_V, _V, _I]),
            "tt_relu": (_V, [_V]), "tt_softmax": (_V, [_V]),
            "tt_conv2d": (_V, [_V, _V, _V, _I, _I, _I, _I]),
            "tt_maxpool2d": (_V, [_V, _I, _I, _I, _I]), "tt_avgpool2d": (_V, [_V, _I, _I, _I, _I]),
            "tt_sgemm_rowmajor": (_I, [_I, _I, _I, _V, _V, _V, _I]),
            "ag_leaf": (_V, [_V, _I]), "ag_matmul": (_V, [_V, _V]), "ag_relu": (_V, [_V]),
            "ag_softmax": (_V, [_V]), "ag_padones": (_V, [_V]),
            "ag_reshape": (_V, [_V, I64P, _I]), "ag_conv2d": (_V, [_V, _V, _V, _I, _I, _I, _I]),
            "ag_maxpool2d": (_V, [_V, _I, _I, _I, _I]), "ag_avgpool2d": (_V, [_V, _I, _I, _I, _I]),
            "ag_value": (_V, [_V]), "ag_grad": (_V, [_V]),
            "ag_backward_from": (None, [_V, F32P, ctypes.c_size_t]),
            "ag_release": (None, [_V]),
        }
        for name, (res, args) in sig.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _REF = h
    return _REF


# ---------------- numpy-level helpers over the restatement ----------------

def sgemm(A, B, nthreads=8):
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    assert orc().orc_sgemm(M, N, K, _p(A), _p(B), _p(C), nthreads) == 0
    return C


def matmul_naive(A, B):
    """reference tt_matmul (src/ops.c:84-101): serial k, zeros of A skipped"""
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    orc().orc_matmul_naive(M, N, K, _p(A), _p(B), _p(C))
    return C


def ref_matmul(A, B):
    """the reference's own tt_matmul, built from its sources"""
    ta, tb = _rt(A), _rt(B)
    o = ref().tt_matmul(ta, tb)
    assert o, "reference tt_matmul returned NULL"
    out = _rnp(o, (A.shape[0], B.shape[1]))
    for t in (ta, tb, o):
        ref().tt_release(t)
    return out


def matmul_nt(X, Y):
    X, Y = f32(X), f32(Y)
    M, K = X.shape
    N = Y.shape[0]
    R = np.empty((M, N), np.float32)
    orc().orc_matmul_nt(M, N, K, _p(X), _p(Y), _p(R))
    return R


def matmul_tn(X, Y):
    X, Y = f32(X), f32(Y)
    K, M = X.shape
    N = Y.shape[1]
    R = np.empty((M, N), np.float32)
    orc().orc_matmul_tn(M, N, K, _p(X), _p(Y), _p(R))
    return R


def sgemm_a_bt(A, B):
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[0]
    C = np.empty((M, N), np.float32)
    orc().orc_sgemm_a_bt(M, N, K, _p(A), _p(B), _p(C))
    return C


def conv_out(H, W, HH, WW, sh, sw, ph, pw):
    return (H + 2 * ph - HH) // sh + 1, (W + 2 * pw - WW) // sw + 1


def im2col(x, HH, WW, sh, sw, ph, pw):
    x = f32(x)
    N, C, H, W = x.shape
    Ho, Wo = conv_out(H, W, HH, WW, sh, sw, ph, pw)
    col = np.empty((C * HH * WW, N * Ho * Wo), np.float32)
    orc().orc_im2col(_p(x), N, C, H, W, HH, WW, ph, pw, sh, sw, _p(col))
    return col


def col2im(col, shape, HH, WW, sh, sw, ph, pw):
    col = f32(col)
    N, C, H, W = shape
    x = np.empty(shape, np.float32)
    orc().orc_col2im(_p(col), N, C, H, W, HH, WW, ph, pw, sh, sw, _p(x))
    return x


def conv2d_fwd(x, w, b, sh, sw, ph, pw, nthreads=8):
    x, w = f32(x), f32(w)
    b = None if b is None else f32(b)
    N, C, H, W = x.shape
    F, _, HH, WW = w.shape
    Ho, Wo = conv_out(H, W, HH, WW, sh, sw, ph, pw)
    out = np.empty((N, F, Ho, Wo), np.float32)
    assert orc().orc_conv2d_fwd(_p(x), N, C, H, W, _p(w), F, HH, WW, _p(b), sh, sw, ph, pw,
                                _p(out), nthreads) == 0
    return out


def conv2d_bwd(x, w, g, sh, sw, ph, pw, need_dx=True, need_dw=True, need_db=True, nthreads=8):
    x, w, g = f32(x), f32(w), f32(g)
    N, C, H, W = x.shape
    F, _, HH, WW = w.shape
    dx = np.empty_like(x) if need_dx else None
    dw = np.empty_like(w) if need_dw else None
    db = np.empty(F, np.float32) if need_db else None
    assert orc().orc_conv2d_bwd(_p(x), N, C, H, W, _p(w), F, HH, WW, _p(g), sh, sw, ph, pw,
                                _p(dx), _p(dw), _p(db), nthreads) == 0
    return dx, dw, db


def bias_grad(g):
    g = f32(g)
    N, F = g.shape[:2]
    HW = int(np.prod(g.shape[2:]))
    db = np.empty(F, np.float32)
    orc().orc_bias_grad(_p(g), N, F, HW, _p(db))
    return db


def pool_out(H, W, ph, pw, sh, sw):
    return (H - ph) // sh + 1, (W - pw) // sw + 1


def maxpool_fwd(x, ph, pw, sh, sw):
    x = f32(x)
    N, C, H, W = x.shape
    Ho, Wo = pool_out(H, W, ph, pw, sh, sw)
    y = np.empty((N, C, Ho, Wo), np.float32)
    orc().orc_maxpool_fwd(_p(x), N, C, H, W, ph, pw, sh, sw, _p(y))
    return y


def maxpool_bwd(x, g, ph, pw, sh, sw):
    x, g = f32(x), f32(g)
    N, C, H, W = x.shape
    dx = np.empty_like(x)
    orc().orc_maxpool_bwd(_p(x), _p(g), N, C, H, W, ph, pw, sh, sw, _p(dx))
    return dx


def avgpool_fwd(x, ph, pw, sh, sw):
    x = f32(x)
    N, C, H, W = x.shape
    Ho, Wo = pool_out(H, W, ph, pw, sh, sw)
    y = np.empty((N, C, Ho, Wo), np.float32)
    orc().orc_avgpool_fwd(_p(x), N, C, H, W, ph, pw, sh, sw, _p(y))
    return y


def avgpool_bwd(g, xshape, ph, pw, sh, sw):
    g = f32(g)
    N, C, H, W = xshape
    dx = np.empty(xshape, np.float32)
    orc().orc_avgpool_bwd(_p(g), N, C, H, W, ph, pw, sh, sw, _p(dx))
    return dx


def relu_fwd(x):
    x = f32(x)
    y = np.empty_like(x)
    orc().orc_relu_fwd(_p(x), _p(y), x.size)
    return y


def relu_bwd(x, g):
    x, g = f32(x), f32(g)
    dx = np.empty_like(x)
    orc().orc_relu_bwd(_p(x), _p(g), _p(dx), x.size)
    return dx


def softmax_fwd(x):
    x = f32(x)
    cols = x.shape[-1]
    y = np.empty_like(x)
    orc().orc_softmax_fwd(_p(x), _p(y), x.size // cols, cols)
    return y


def softmax_bwd(s, g):
    s, g = f32(s), f32(g)
    cols = s.shape[-1]
    dx = np.empty_like(s)
    orc().orc_softmax_bwd(_p(s), _p(g), _p(dx), s.size // cols, cols)
    return dx


def padones_fwd(x):
    x = f32(x)
    M, K = x.shape
    y = np.empty((M, K + 1), np.float32)
    orc().orc_padones_fwd(_p(x), _p(y), M, K)
    return y


def padones_bwd(g):
    g = f32(g)
    M, K1 = g.shape
    dx = np.empty((M, K1 - 1), np.float32)
    orc().orc_padones_bwd(_p(g), _p(dx), M, K1 - 1)
    return dx


def ce_seed(p, labels):
    p = f32(p)
    lab = np.ascontiguousarray(labels, dtype=np.int32)
    rows, cols = p.shape
    seed = np.empty_like(p)
    loss = orc().orc_ce_seed(_p(p), _p(lab), rows, cols, _p(seed))
    return loss, seed


def momentum_step(w, v, g, lr, mu):
    """SGD with momentum of the reference MNIST harness (reference
    tests/gate_mnist_mlp.py:121-124): v = mu*v - lr*g, then w = w + v, on
    float32 arrays with Python-float hyperparameters.  NumPy 2 rounds a
    Python float to float32 against a float32 array, and every product is
    rounded before the subtraction.  Updates w and v in place."""
    assert w.dtype == v.dtype == g.dtype == np.float32
    v[:] = np.float32(mu) * v - np.float32(lr) * g
    w[:] = w + v


def adam_lr_t(lr, b1, b2, t):
    """Bias-corrected step size of step t (reference tests/gate_cifar_cnn.py:93-94),
    a float64."""
    return lr * (math.sqrt(1.0 - b2 ** t) / (1.0 - b1 ** t))


def adam_step(params, grads, m, v, t, lr=0.003, b1=0.9, b2=0.999, eps=1e-8):
    """Step t (1-based) of the reference CIFAR harness's Adam (reference
    tests/gate_cifar_cnn.py:81-98) with its dtypes written out: the moments
    are float32 (the Python-float betas rounded to float32), the step
    lr_t*m/(sqrt(v)+eps) is float64 because lr_t is a NumPy float64 scalar,
    and the in-place subtraction rounds the float64 result into the float32
    parameter once.  Updates params, m and v in place."""
    lr_t = adam_lr_t(lr, b1, b2, t)
    c1, d1 = np.float32(b1), np.float32(1.0 - b1)
    c2, d2 = np.float32(b2), np.float32(1.0 - b2)
    for p, g, mi, vi in zip(params, grads, m, v):
        mi[:] = c1 * mi + d1 * g
        vi[:] = c2 * vi + d2 * (g * g)
        den = (np.sqrt(vi) + np.float32(eps)).astype(np.float64)
        p[:] = (p.astype(np.float64) - (lr_t * mi.astype(np.float64)) / den).astype(np.float32)


def read_idx(path):
    """uint8 idx file (gzip'd or plain) -> ndarray of its dims.  The MNIST
    harness's parse (reference tests/gate_mnist_mlp.py:44-53): big-endian
    header (0, 0, type 0x08, ndim) then ndim uint32 dims, data after."""
    import gzip
    with open(path, "rb") as f:
        raw = f.read()
    if raw[:2] == b"\x1f\x8b":
        raw = gzip.decompress(raw)
    assert raw[0] == 0 and raw[1] == 0 and raw[2] == 0x08, "not a uint8 idx file"
    nd = raw[3]
    dims = [int.from_bytes(raw[4 + 4 * i: 8 + 4 * i], "big") for i in range(nd)]
    off = 4 + 4 * nd
    return np.frombuffer(raw, np.uint8, count=int(np.prod(dims)), offset=off).reshape(dims)


def read_cifar_bin(paths):
    """CIFAR-10 binary batches -> (uint8 (n, 3, 32, 32), int32 labels): records
    of 1 label byte + 3072 channel-major pixels, files concatenated."""
    recs = np.concatenate([np.fromfile(p, np.uint8).reshape(-1, 3073) for p in paths])
    return recs[:, 1:].reshape(-1, 3, 32, 32).copy(), recs[:, 0].astype(np.int32)


def normalize_u8(x, mean, std):
    """((x / 255) - mean[c]) / std[c] in float32, channel axis 1 -- the
    harnesses' normalisation (reference tests/gate_mnist_mlp.py:85,
    tests/gate_cifar_cnn.py:165) with the float32 scalars written out."""
    x = x.astype(np.float32) / np.float32(255.0)
    m = np.asarray(mean, np.float32).reshape((1, -1) + (1,) * (x.ndim - 2))
    s = np.asarray(std, np.float32).reshape((1, -1) + (1,) * (x.ndim - 2))
    return (x - m) / s


def mlp_step(x, labels, W1, W2, W3, nthreads=8):
    x, W1, W2, W3 = f32(x), f32(W1), f32(W2), f32(W3)
    lab = np.ascontiguousarray(labels, dtype=np.int32)
    B, d0 = x.shape
    d1, d2, d3 = W1.shape[1], W2.shape[1], W3.shape[1]
    logits = np.empty((B, d3), np.float32)
    probs = np.empty_like(logits)
    g1, g2, g3 = np.empty_like(W1), np.empty_like(W2), np.empty_like(W3)
    loss = orc().orc_mlp_step(B, d0, d1, d2, d3, _p(x), _p(lab), _p(W1), _p(W2), _p(W3),
                              _p(logits), _p(probs), _p(g1), _p(g2), _p(g3), nthreads)
    return dict(loss=loss, logits=logits, probs=probs, dW1=g1, dW2=g2, dW3=g3)


def cnn_step(x, labels, w1, b1, w2, b2, wfc, nthreads=8):
    x, w1, b1, w2, b2, wfc = map(f32, (x, w1, b1, w2, b2, wfc))
    lab = np.ascontiguousarray(labels, dtype=np.int32)
    B, C0, H, W = x.shape
    F1, F2, classes = w1.shape[0], w2.shape[0], wfc.shape[1]
    logits = np.empty((B, classes), np.float32)
    probs = np.empty_like(logits)
    out = dict(dw1=np.empty_like(w1), db1=np.empty_like(b1), dw2=np.empty_like(w2),
               db2=np.empty_like(b2), dwfc=np.empty_like(wfc))
    loss = orc().orc_cnn_step(B, C0, H, W, F1, F2, classes, _p(x), _p(lab), _p(w1), _p(b1),
                              _p(w2), _p(b2), _p(wfc), _p(logits), _p(probs), _p(out["dw1"]),
                              _p(out["db1"]), _p(out["dw2"]), _p(out["db2"]), _p(out["dwfc"]),
                              nthreads)
    out.update(loss=loss, logits=logits, probs=probs)
    return out


def uniform(shape, lo, hi, seed):
    a = np.empty(int(np.prod(shape)), np.float32)
    orc().orc_fill_uniform(_p(a), a.size, lo, hi, seed)
    return a.reshape(shape)


def normal(shape, std, seed):
    a = np.empty(int(np.prod(shape)), np.float32)
    orc().orc_fill_normal(_p(a), a.size, std, seed)
    return a.reshape(shape)


def labels(n, classes, seed):
    a = np.empty(n, np.int32)
    orc().orc_fill_labels(_p(a), n, classes, seed)
    return a


# ---------------- configs of BASELINE.json (seeded synthetic inputs) ----------------

def mlp_inputs(B=256, dims=(784, 512, 256, 10), seed=0x5EED):
    d0, d1, d2, d3 = dims
    x = uniform((B, d0), 0.0, 1.0, seed + 1)
    y = labels(B, d3, seed + 2)
    Ws = []
    for i, (fi, fo) in enumerate(((d0, d1), (d1, d2), (d2, d3))):
        w = normal((fi + 1, fo), float(np.sqrt(2.0 / fi)), seed + 10 + i)
        w[fi, :] = 0.0  # bias row (padones) starts at zero
        Ws.append(w)
    return x, y, Ws


def cnn_inputs(B=128, C0=3, H=32, W=32, F1=32, F2=64, classes=10, seed=0x5EED):
    x = uniform((B, C0, H, W), 0.0, 1.0, seed + 1)
    y = labels(B, classes, seed + 2)
    w1 = normal((F1, C0, 3, 3), float(np.sqrt(2.0 / (C0 * 9))), seed + 10)
    b1 = np.zeros(F1, np.float32)
    w2 = normal((F2, F1, 3, 3), float(np.sqrt(2.0 / (F1 * 9))), seed + 11)
    b2 = np.zeros(F2, np.float32)
    D = F2 * (H // 4) * (W // 4)
    wfc = normal((D + 1, classes), float(np.sqrt(2.0 / D)), seed + 12)
    wfc[D, :] = 0.0
    return x, y, dict(w1=w1, b1=b1, w2=w2, b2=b2, wfc=wfc)


# ---------------- the reference library itself (oracle/_ref) ----------------
# Used to pin the restatement above and as the "reference" CPU baseline.

def _rt(a):
    """numpy -> reference Tensor* (owned)."""
    a = f32(a)
    shp = (ctypes.c_long * a.ndim)(*a.shape)
    t = ref().tt_fromdata(a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), shp, a.ndim)
    assert t, "reference tt_fromdata failed"
    return t


def _rnp(t, shape):
    n = int(np.prod(shape))
    buf = np.ctypeslib.as_array(ref().tt_data(t), shape=(n,))
    return buf.copy().reshape(shape)


class RefGraph:
    """Builds a graph on the reference autograd and releases it afterwards."""

    def __init__(self):
        self.nodes = []

    def leaf(self, a, req=True):
        t = _rt(a)
        n = ref().ag_leaf(t, 1 if req else 0)
        ref().tt_release(t)
        self.nodes.append(n)
        return n

    def add(self, n):
        assert n, "reference op returned NULL"
        self.nodes.append(n)
        return n

    def value(self, n, shape):
        return _rnp(ref().ag_value(n), shape)

    def grad(self, n, shape):
        g = ref().ag_grad(n)
        return None if not g else _rnp(g, shape)

    def backward(self, n, seed):
        seed = f32(seed)
        ref().ag_backward_from(n, seed.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), seed.size)

    def release(self):
        for n in self.nodes:
            ref().ag_release(n)
        self.nodes = []


def ref_sgemm(A, B, nthreads=8):
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.zeros((M, N), np.float32)
    assert ref().tt_sgemm_rowmajor(M, N, K, _p(A), _p(B), _p(C), nthreads) == 0
    return C


def ref_unary(name, x, *args):
    t = _rt(x)
    o = getattr(ref(), name)(t, *args)
    assert o, f"reference {name} returned NULL"
    n = int(ref().tt_numel(o))
    out = np.ctypeslib.as_array(ref().tt_data(o), shape=(n,)).copy()
    ref().tt_release(t)
    ref().tt_release(o)
    return out


def ref_cnn_step(x, labels, w1, b1, w2, b2, wfc):
    """The reference autograd path of the CNN config: forward, softmax, CE
    seed in NumPy, backward (tests/gate_cifar_cnn.py:165-186 pattern)."""
    g = RefGraph()
    B = x.shape[0]
    L = ref()
    X = g.leaf(x, False)
    n_w1, n_b1, n_w2, n_b2, n_fc = (g.leaf(a) for a in (w1, b1, w2, b2, wfc))
    h = g.add(L.ag_conv2d(X, n_w1, n_b1, 1, 1, 1, 1))
    h = g.add(L.ag_relu(h))
    h = g.add(L.ag_maxpool2d(h, 2, 2, 2, 2))
    h = g.add(L.ag_conv2d(h, n_w2, n_b2, 1, 1, 1, 1))
    h = g.add(L.ag_relu(h))
    h = g.add(L.ag_maxpool2d(h, 2, 2, 2, 2))
    D = int(np.prod(wfc.shape[0] - 1))
    shp = (ctypes.c_long * 2)(B, D)
    h = g.add(L.ag_reshape(h, shp, 2))
    h = g.add(L.ag_padones(h))
    logits = g.add(L.ag_matmul(h, n_fc))
    probs_n = g.add(L.ag_softmax(logits))
    classes = wfc.shape[1]
    p = g.value(probs_n, (B, classes))
    onehot = np.zeros((B, classes), np.float32)
    onehot[np.arange(B), labels] = 1.0
    g.backward(logits, (p - onehot) / float(B))
    out = dict(logits=g.value(logits, (B, classes)), probs=p,
               dw1=g.grad(n_w1, w1.shape), db1=g.grad(n_b1, b1.shape),
               dw2=g.grad(n_w2, w2.shape), db2=g.grad(n_b2, b2.shape),
               dwfc=g.grad(n_fc, wfc.shape))
    g.release()
    return out


def ref_mlp_step(x, labels, W1, W2, W3):
    """The reference autograd path of the MLP config (tests/gate_mnist_mlp.py:68-71,108-119)."""
    g = RefGraph()
    L = ref()
    B = x.shape[0]
    X = g.leaf(x, False)
    n1, n2, n3 = g.leaf(W1), g.leaf(W2), g.leaf(W3)
    h = g.add(L.ag_padones(X))
    h = g.add(L.ag_relu(g.add(L.ag_matmul(h, n1))))
    h = g.add(L.ag_padones(h))
    h = g.add(L.ag_relu(g.add(L.ag_matmul(h, n2))))
    h = g.add(L.ag_padones(h))
    logits = g.add(L.ag_matmul(h, n3))
    probs_n = g.add(L.ag_softmax(logits))
    classes = W3.shape[1]
    p = g.value(probs_n, (B, classes))
    onehot = np.zeros((B, classes), np.float32)
    onehot[np.arange(B), labels] = 1.0
    g.backward(logits, (p - onehot) / float(B))
    out = dict(logits=g.value(logits, (B, classes)), probs=p, dW1=g.grad(n1, W1.shape),
               dW2=g.grad(n2, W2.shape), dW3=g.grad(n3, W3.shape))
    g.release()
    return out
