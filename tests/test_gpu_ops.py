"""The tt_* tensor C ABI on the GPU, following the reference's own op tests
(reference tests/test_ops.py): ops against NumPy closed forms and the
oracle, shape/stride metadata, NULL on bad arguments, the hostile-parameter
and NaN/Inf battery, reshape-is-a-copy, and the host-mirror contract of
tt_data."""
import ctypes

import numpy as np
import pytest

import orc
import tinytorch_amd
from tinytorch_amd import F32P

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(42)


@pytest.fixture(scope="module")
def L(tlib):
    return tlib


def make(L, arr):
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    shape = (ctypes.c_long * max(arr.ndim, 1))(*arr.shape)
    t = L.tt_fromdata(arr.ctypes.data_as(F32P), shape, arr.ndim)
    assert t, f"tt_fromdata failed for {arr.shape}"
    return t


def to_np(L, t, shape):
    n = int(L.tt_numel(t))
    return np.ctypeslib.as_array(L.tt_data(t), shape=(n,)).copy().reshape(shape)


def shape_of(L, t):
    nd = L.tt_ndim(t)
    s = (ctypes.c_long * nd)()
    L.tt_shape(t, s)
    return tuple(s)


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("shape", [(8,), (3, 4), (2, 3, 4), (1000, 17)])
def test_elementwise(L, shape):
    x = rng.standard_normal(shape).astype(np.float32)
    y = rng.standard_normal(shape).astype(np.float32)
    tx, ty = make(L, x), make(L, y)
    for fn, ref in ((L.tt_add, x + y), (L.tt_mul, x * y)):
        o = fn(tx, ty)
        assert bits_equal(to_np(L, o, shape), ref)
        L.tt_release(o)
    for fn, s, ref in ((L.tt_addscalar, 2.5, x + np.float32(2.5)),
                       (L.tt_mulscalar, -0.5, x * np.float32(-0.5))):
        o = fn(tx, ctypes.c_float(s))
        assert bits_equal(to_np(L, o, shape), ref)
        L.tt_release(o)
    o = L.tt_relu(tx)
    assert bits_equal(to_np(L, o, shape), np.maximum(x, 0.0))
    L.tt_release(o)
    L.tt_release(tx)
    L.tt_release(ty)


@pytest.mark.parametrize("sa,sb", [((3, 4), (4, 5)), ((16, 16), (16, 16)), ((1, 7), (7, 1)),
                                   ((32, 64), (64, 17)), ((17, 13), (13, 5)), ((7, 7), (7, 7)),
                                   ((5, 300), (300, 3)), ((9, 256), (256, 33)),
                                   ((64, 512), (512, 16))])
def test_matmul_variants(L, sa, sb):
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    ref = a.astype(np.float64) @ b
    ta, tb = make(L, a), make(L, b)
    for fn in (L.tt_matmul, L.tt_matmul_fast, lambda x, y: L.tt_matmul_omp(x, y, 4)):
        o = fn(ta, tb)
        got = to_np(L, o, ref.shape)
        assert np.allclose(got, ref, atol=1e-4, rtol=1e-4)
        assert np.abs(got - orc.sgemm(a, b)).max() <= 1e-4 * np.sqrt(sa[1]) * np.abs(a).max() * np.abs(b).max()
        L.tt_release(o)
    L.tt_release(ta)
    L.tt_release(tb)


@pytest.mark.parametrize("M,N,K", [(37, 45, 29), (36, 48, 29), (5, 40, 9), (40, 15, 9),
                                   (12, 32, 0), (1, 1, 3)])
def test_sgemm_rowmajor_host_pointers(L, M, N, K):
    """C on entry is overwritten on the reference's main block and
    accumulated into everywhere else (src/gemm.c:569-641): compared with the
    reference build itself where it exists, else with the oracle."""
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = rng.uniform(2, 3, (M, N)).astype(np.float32)
    C = C0.copy()
    assert L.tt_sgemm_rowmajor(M, N, K, A.ctypes.data_as(F32P), B.ctypes.data_as(F32P),
                               C.ctypes.data_as(F32P), 6) == 0
    mb, nb = M // 6 * 6, N // 16 * 16
    keep = np.ones((M, N))
    if K > 0 and mb and nb:   # main block overwritten, the rest accumulated
        keep[:mb, :nb] = 0.0
    want = A.astype(np.float64) @ B + keep * C0
    assert np.abs(C - want).max() <= 1e-4 * np.sqrt(max(K, 1)) * 4
    if K == 0:
        assert np.array_equal(C, C0)
    if orc.ref_available():   # the reference build on the same C
        R = C0.copy()
        assert orc.ref().tt_sgemm_rowmajor(M, N, K, A.ctypes.data, B.ctypes.data, R.ctypes.data,
                                           1) == 0
        assert np.abs(C - R).max() <= 1e-4 * np.sqrt(max(K, 1)) * 4


def test_matmul_naive_bitexact_and_zero_skip(L):
    """tt_matmul keeps the reference's naive arithmetic (src/ops.c:84-101):
    bit-identical to the oracle, a zero of A masks NaN / Inf in B."""
    M, N, K = 37, 300, 23
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    A[A < -0.6] = 0.0
    A[1, 2] = -0.0
    A[3, 2] = 0.5
    B[2, :5] = [np.nan, np.inf, -np.inf, np.nan, 1.0]
    ta, tb = make(L, A), make(L, B)
    o = L.tt_matmul(ta, tb)
    got = to_np(L, o, (M, N))
    assert bits_equal(got, orc.matmul_naive(A, B))
    assert np.isfinite(got[1]).all() and np.isnan(got[3, 0])
    for t in (o, ta, tb):
        L.tt_release(t)


def softmax_ref(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("x", [rng.standard_normal((5,)), rng.standard_normal((3, 6)),
                               rng.standard_normal((2, 3, 4)) + 100.0,
                               np.full((4,), -1e9), rng.standard_normal((4, 100))])
def test_softmax(L, x):
    x = x.astype(np.float32)
    t = make(L, x)
    o = L.tt_softmax(t)
    got = to_np(L, o, x.shape)
    assert np.allclose(got, softmax_ref(x), atol=1e-5, rtol=1e-5)
    assert np.allclose(got.sum(axis=-1), 1.0, atol=1e-5)
    L.tt_release(o)
    L.tt_release(t)


def test_softmax_all_neginf_uniform(L):
    x = np.array([[-np.inf] * 4, [1.0, 2.0, 3.0, 4.0]], np.float32)
    t = make(L, x)
    o = L.tt_softmax(t)
    got = to_np(L, o, x.shape)
    assert np.all(got[0] == 0.25) and not np.isnan(got).any()
    assert np.allclose(got[1], softmax_ref(x[1:])[0], atol=1e-5, rtol=1e-5)
    L.tt_release(o)
    L.tt_release(t)


def test_metadata_and_errors(L):
    x = rng.standard_normal((2, 3, 4)).astype(np.float32)
    t = make(L, x)
    st = (ctypes.c_long * 3)()
    L.tt_strides(t, st)
    assert shape_of(L, t) == (2, 3, 4) and list(st) == [12, 4, 1]
    assert L.tt_ndim(t) == 3 and L.tt_numel(t) == 24
    a, b = make(L, np.ones((3, 4))), make(L, np.ones((5, 6)))
    c = make(L, np.ones((2, 3)))
    assert not L.tt_matmul(a, b) and not L.tt_matmul_fast(a, b) and not L.tt_add(a, c)
    for h in (t, a, b, c):
        L.tt_release(h)
    u = L.tt_retain(None)
    assert not u


def test_new_is_zero_filled(L):
    shp = (ctypes.c_long * 2)(300, 301)
    t = L.tt_new(shp, 2)
    assert t and np.all(to_np(L, t, (300, 301)) == 0.0)
    L.tt_release(t)


def test_host_writes_through_tt_data_are_seen(L):
    """tt_data hands out a host pointer the caller may write; the next op
    uploads it (the reference's tensors are plain host memory)."""
    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    t = make(L, x)
    p = L.tt_data(t)
    p[0] = -5.0
    o = L.tt_relu(t)
    assert to_np(L, o, (2, 3)).ravel().tolist() == [0, 1, 2, 3, 4, 5]
    L.tt_release(o)
    L.tt_release(t)


def test_hostile_conv_pool_params(L):
    a, w = make(L, rng.standard_normal((1, 1, 8, 8))), make(L, rng.standard_normal((2, 1, 3, 3)))
    assert not L.tt_conv2d(a, w, None, 0, 1, 0, 0)
    assert not L.tt_conv2d(a, w, None, -1, 1, 0, 0)
    assert not L.tt_conv2d(a, w, None, 1, 1, -1, 0)
    assert not L.tt_maxpool2d(a, 0, 2, 2, 2)
    assert not L.tt_avgpool2d(a, 2, 2, 0, 2)

    class CT(ctypes.Structure):
        _fields_ = [("data", F32P), ("shape", ctypes.POINTER(ctypes.c_long)),
                    ("strides", ctypes.POINTER(ctypes.c_long)), ("ndim", ctypes.c_int),
                    ("numel", ctypes.c_long), ("refcount", ctypes.c_int)]
    tw = CT.from_address(w)
    assert tw.ndim == 4 and tw.shape[2] == 3
    tw.shape[2] = 0  # HH = 0 poked through the public layout
    assert not L.tt_conv2d(a, w, None, 1, 1, 0, 0)
    tw.shape[2] = 3
    bad_b = make(L, np.ones(3))
    assert not L.tt_conv2d(a, w, bad_b, 1, 1, 1, 1)  # bias length != F
    for h in (a, w, bad_b):
        L.tt_release(h)


def test_nan_inf_inputs_no_crash(L):
    for arr in (np.array([np.nan, 1.0, -2.0]), np.array([np.inf, -np.inf, 1.5]),
                np.array([1.0, np.inf, -np.inf, 0.0])):
        t = make(L, arr)
        for fn in (L.tt_relu, L.tt_softmax):
            o = fn(t)
            assert o
            L.tt_release(o)
        L.tt_release(t)
    m1, m2 = make(L, np.full((4, 4), np.nan)), make(L, np.ones((4, 4)))
    o = L.tt_matmul(m1, m2)
    assert o and np.isnan(to_np(L, o, (4, 4))).all()
    for h in (o, m1, m2):
        L.tt_release(h)


@pytest.mark.parametrize("v,want", [(-2e30, np.float32(-2e30)), (-np.inf, -np.inf), (np.nan, -np.inf)])
def test_maxpool_special_values(L, v, want):
    t = make(L, np.full((1, 1, 4, 4), v, np.float32))
    o = L.tt_maxpool2d(t, 2, 2, 2, 2)
    got = to_np(L, o, (1, 1, 2, 2))
    assert np.all(got == want) and not np.isnan(got).any()
    L.tt_release(o)
    L.tt_release(t)


def test_reshape_is_a_copy(L):
    x = np.arange(12, dtype=np.float32).reshape(2, 6)
    t = make(L, x)
    ns = (ctypes.c_long * 2)(3, 4)
    o = L.tt_reshape(t, ns, 2)
    assert o
    assert ctypes.cast(L.tt_data(o), ctypes.c_void_p).value != ctypes.cast(L.tt_data(t), ctypes.c_void_p).value
    assert np.array_equal(to_np(L, o, (3, 4)), x.reshape(3, 4))
    st = (ctypes.c_long * 2)()
    L.tt_strides(o, st)
    assert tuple(st) == (4, 1)
    bad = (ctypes.c_long * 2)(5, 5)
    assert not L.tt_reshape(t, bad, 2)
    L.tt_release(o)
    L.tt_release(t)


@pytest.mark.parametrize("sh,ph", [(1, 1), (2, 0), (1, 2)])
def test_conv_and_pools_vs_oracle(L, sh, ph):
    x = rng.standard_normal((3, 4, 10, 9)).astype(np.float32)
    w = rng.standard_normal((6, 4, 3, 3)).astype(np.float32)
    b = rng.standard_normal(6).astype(np.float32)
    tx, tw, tb = make(L, x), make(L, w), make(L, b)
    ref = orc.conv2d_fwd(x, w, b, sh, sh, ph, ph)
    o = L.tt_conv2d(tx, tw, tb, sh, sh, ph, ph)
    got = to_np(L, o, ref.shape)
    assert np.abs(got - ref).max() <= 1e-4 * np.sqrt(36) * np.abs(x).max() * np.abs(w).max()
    L.tt_release(o)
    o = L.tt_conv2d(tx, tw, None, sh, sh, ph, ph)  # no bias
    assert np.abs(to_np(L, o, ref.shape) - (ref - b[None, :, None, None])).max() < 1e-3
    L.tt_release(o)
    for p, s in ((2, 2), (3, 2)):
        o = L.tt_maxpool2d(tx, p, p, s, s)
        want = orc.maxpool_fwd(x, p, p, s, s)
        assert bits_equal(to_np(L, o, want.shape), want)
        L.tt_release(o)
        o = L.tt_avgpool2d(tx, p, p, s, s)
        want = orc.avgpool_fwd(x, p, p, s, s)
        assert bits_equal(to_np(L, o, want.shape), want)
        L.tt_release(o)
    for h in (tx, tw, tb):
        L.tt_release(h)


def test_retain_release_10k(L):
    t = make(L, np.ones(8))
    for _ in range(10000):
        u = L.tt_retain(t)
        assert u
        L.tt_release(u)
    L.tt_release(t)


def test_allocator_reuses_blocks(L):
    before = L.tth_bytes_in_use()
    for _ in range(50):
        t = make(L, np.ones((256, 1024)))
        L.tt_release(t)
    assert L.tth_bytes_in_use() == before
    assert tinytorch_amd.device_name().startswith("gfx950")


def _bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("M,K", [(1, 1), (128, 4096), (3, 1023), (7, 1024), (5, 3000)])
def test_copy_padones_kernel_bitexact(tlib, M, K):
    """tt_k_copy_padones_fwd: the copy and the padded tensor bit for bit
    equal to tt_k_copy + tt_k_padones_fwd (reference src/ops_spatial.c:22-34,
    src/autograd.c:195-212)."""
    from tinytorch_amd.hip import DevBuf, check
    x = rng.standard_normal((M, K)).astype(np.float32)
    x.flat[::5] = np.nan
    dx_, c1, y1, c2, y2 = (DevBuf.from_np(x), DevBuf(M * K), DevBuf(M * (K + 1)), DevBuf(M * K),
                           DevBuf(M * (K + 1)))
    check(tlib.tt_k_copy_padones_fwd(dx_.ptr, c1.ptr, y1.ptr, M, K), "copy_padones")
    check(tlib.tt_k_copy(c2.ptr, dx_.ptr, M * K), "copy")
    check(tlib.tt_k_padones_fwd(dx_.ptr, y2.ptr, M, K), "padones")
    assert _bits(c1.to_np((M, K)), c2.to_np((M, K)))
    assert _bits(y1.to_np((M, K + 1)), y2.to_np((M, K + 1)))
    assert _bits(y1.to_np((M, K + 1))[:, K], np.ones(M, np.float32))


@pytest.mark.parametrize("mode", ["fused", "peek", "other"])
def test_autograd_reshape_padones_deferred(tlib, mode):
    """ag_reshape followed by ag_padones (one launch) against the same graph
    with deferral off: values and gradients bit for bit equal; reading the
    reshape's value first, or another op in between, launches the pending
    copy first."""
    from tinytorch_amd.torch_py import Node
    x = rng.standard_normal((16, 8, 4, 4)).astype(np.float32)
    # 40 columns: above the fused classifier head's limit (32), whose
    # backward sums in another order than the GEMM path this compares with
    w = rng.standard_normal((129, 40)).astype(np.float32)
    g = rng.standard_normal((16, 40)).astype(np.float32)

    def run(m):
        X, Wn = Node.leaf(x), Node.leaf(w)
        r = X.reshape((16, 128))
        if m == "peek":
            rv = r.value()
        if m == "other":
            o = Wn.relu()
            o.release()
        p = r.padones()
        out = p.matmul(Wn)
        vals = [r.value(), p.value(), out.value()]
        out.backward(g)
        res = vals + [X.grad(), Wn.grad()]
        if m == "peek":
            assert _bits(rv, vals[0])
        for n in (out, p, r, X, Wn):
            n.release()
        return res

    prev = tlib.tth_conv_relu_fuse(0)
    try:
        ref = run("plain")
    finally:
        tlib.tth_conv_relu_fuse(prev)
    for a, e in zip(run(mode), ref):
        assert _bits(a, e), mode
    assert _bits(ref[0], x.reshape(16, 128))


@pytest.mark.parametrize("M,K", [(1, 1), (256, 512), (3, 1023), (5, 3000)])
def test_relu_padones_kernel_bitexact(tlib, M, K):
    """tt_k_relu_padones_fwd: relu output and padded tensor bit for bit equal
    to tt_k_relu_fwd + tt_k_padones_fwd, NaN and -0 included."""
    from tinytorch_amd.hip import DevBuf, check
    x = rng.standard_normal((M, K)).astype(np.float32)
    x.flat[::5] = np.nan
    x.flat[1::7] = -0.0
    dx_, r1, y1, r2, y2 = (DevBuf.from_np(x), DevBuf(M * K), DevBuf(M * (K + 1)), DevBuf(M * K),
                           DevBuf(M * (K + 1)))
    check(tlib.tt_k_relu_padones_fwd(dx_.ptr, r1.ptr, y1.ptr, M, K), "relu_padones")
    check(tlib.tt_k_relu_fwd(dx_.ptr, r2.ptr, M * K), "relu")
    check(tlib.tt_k_padones_fwd(r2.ptr, y2.ptr, M, K), "padones")
    assert _bits(r1.to_np((M, K)), r2.to_np((M, K)))
    assert _bits(y1.to_np((M, K + 1)), y2.to_np((M, K + 1)))


@pytest.mark.parametrize("mode", ["fused", "peek", "other", "no_padones"])
def test_autograd_relu_padones_deferred(tlib, mode):
    """ag_relu followed by ag_padones (one launch) against deferral off, for
    a two-layer MLP fragment: values and gradients bit for bit equal."""
    from tinytorch_amd.torch_py import Node
    x = rng.standard_normal((32, 20)).astype(np.float32)
    # 40 columns: above the fused classifier head's limit (32), whose
    # backward sums in another order than the GEMM path this compares with
    w1 = rng.standard_normal((21, 40)).astype(np.float32)
    w2 = rng.standard_normal((41, 40)).astype(np.float32)
    g = rng.standard_normal((32, 40)).astype(np.float32)

    def run(m):
        X, W1, W2 = Node.leaf(x), Node.leaf(w1), Node.leaf(w2)
        h = X.padones().matmul(W1)
        r = h.relu()
        if m == "peek":
            rv = r.value()
        if m == "other":
            o = W2.relu()
            o.release()
        if m == "no_padones":
            s_ = r * 2.0            # a consumer other than padones launches the relu first
            sv = s_.value()
            s_.release()
        p = r.padones()
        out = p.matmul(W2)
        vals = [h.value(), r.value(), p.value(), out.value()]
        out.backward(g)
        res = vals + [X.grad(), W1.grad(), W2.grad()]
        if m == "peek":
            assert _bits(rv, vals[1])
        if m == "no_padones":
            assert _bits(sv, vals[1] * np.float32(2.0))
        for n in (out, p, r, h, X, W1, W2):
            n.release()
        return res

    prev = tlib.tth_conv_relu_fuse(0)
    try:
        ref = run("plain")
    finally:
        tlib.tth_conv_relu_fuse(prev)
    for a, e in zip(run(mode), ref):
        assert _bits(a, e), mode


@pytest.mark.parametrize("shared", [False, True])
def test_padones_backward_through_reshape(tlib, shared):
    """reshape -> padones -> matmul: the reshape's gradient is the padones
    backward (g without its last column) and its input's gradient the same
    values in the input's shape, bit for bit, whether written by the one-pass
    form (reshape used once) or by the separate passes (reshape shared)."""
    from tinytorch_amd.torch_py import Node
    x = rng.standard_normal((8, 4, 2, 3)).astype(np.float32)
    w = rng.standard_normal((25, 5)).astype(np.float32)
    g = rng.standard_normal((8, 5)).astype(np.float32)
    X, Wn = Node.leaf(x), Node.leaf(w)
    r = X.reshape((8, 24))
    p = r.padones()
    out = p.matmul(Wn)
    if shared:
        # r also feeds a second consumer: the separate passes run
        s_ = r * 1.0
        Z = Node.leaf(np.zeros((5, 24), np.float32), False)
        z = out.matmul(Z)
        tot = z + s_
        G = rng.standard_normal((8, 24)).astype(np.float32)
        tot.backward(G)
        assert _bits(r.grad(), G)
        assert _bits(X.grad(), G.reshape(x.shape))
        for n in (tot, z, Z, s_, out, p, r, X, Wn):
            n.release()
        return
    out.backward(g)
    gp = p.grad()
    assert _bits(r.grad(), gp[:, :24])
    assert _bits(X.grad(), gp[:, :24].reshape(x.shape))
    ref = (g.astype(np.float64) @ w.T.astype(np.float64))[:, :24]
    assert np.abs(r.grad() - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    for n in (out, p, r, X, Wn):
        n.release()
