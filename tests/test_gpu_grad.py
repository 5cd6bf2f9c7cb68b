"""Autograd on the GPU, following the reference's gradcheck gate and its
seed / edge battery (reference tests/test_grad.py): every backward rule
against central finite differences (h = 1e-2, RTOL 1e-4, ATOL 1e-5, conv
ATOL 2e-4), the seed-length contract, ones seeding, dtype coercion, a
1000-deep chain, grad accumulation across backward calls on a shared
subgraph (3x), NaN/Inf safety; plus every rule's gradient against the
oracle's closed-form backward at larger shapes."""
import numpy as np
import pytest

import orc

pytestmark = pytest.mark.gpu

RTOL, ATOL, H = 1e-4, 1e-5, 1e-2


@pytest.fixture(scope="module")
def Node(tlib):
    from tinytorch_amd.torch_py import Node as _Node
    return _Node


rng = np.random.default_rng(0)


def clear_x(shape):
    """random tensor with |x| > 0.05 everywhere (keeps FD off the relu kink)"""
    while True:
        x = rng.standard_normal(shape).astype(np.float32)
        if np.abs(x).min() > 0.05:
            return x


def gradcheck(Node, build, arrays, atol=ATOL):
    probe = [Node.leaf(a.copy(), False) for a in arrays]
    out = build(*probe)
    R = np.random.default_rng(7).standard_normal(out.value().shape).astype(np.float32)
    out.release()
    for n in probe:
        n.release()

    def scalar(arrs):
        nodes = [Node.leaf(a, True) for a in arrs]
        o = build(*nodes)
        v = float(np.sum(R * o.value(), dtype=np.float64))
        return v, nodes, o

    _, nodes, o = scalar([a.copy() for a in arrays])
    o.backward(R)
    analytic = [n.grad().copy() for n in nodes]
    for n in nodes + [o]:
        n.release()
    for k, a in enumerate(arrays):
        num = np.zeros(a.size)
        for i in range(a.size):
            ap = [x.copy() for x in arrays]
            am = [x.copy() for x in arrays]
            ap[k].reshape(-1)[i] += H
            am[k].reshape(-1)[i] -= H
            fp, n1, o1 = scalar(ap)
            fm, n2, o2 = scalar(am)
            for n in n1 + n2 + [o1, o2]:
                n.release()
            num[i] = (fp - fm) / (2 * H)
        viol = np.abs(analytic[k].reshape(-1) - num) - RTOL * np.abs(num)
        assert viol.max() < atol, f"input {k}: violation {viol.max():.3e}"


CASES = {
    "add": (lambda x, y: x + y, [(4, 3), (4, 3)], ATOL),
    "mul": (lambda x, y: x * y, [(4, 3), (4, 3)], ATOL),
    "addscalar": (lambda x: x + 1.5, [(4, 3)], ATOL),
    "mulscalar": (lambda x: x * (-0.7), [(4, 3)], ATOL),
    "relu": (lambda x: x.relu(), [(4, 3)], ATOL),
    "matmul": (lambda x, w: x.matmul(w), [(4, 3), (3, 5)], ATOL),
    "softmax": (lambda x: x.softmax(), [(4, 5)], ATOL),
    "padones": (lambda x: x.padones(), [(4, 3)], ATOL),
    "reshape": (lambda x: x.reshape((2, 6)), [(3, 4)], ATOL),
    "conv2d": (lambda x, w, b: x.conv2d(w, b, stride=1, pad=1), [(2, 2, 5, 5), (3, 2, 3, 3), (3,)], 2e-4),
    "maxpool2d": (lambda x: x.maxpool2d(pool_size=2, stride=2), [(2, 2, 6, 6)], ATOL),
    "avgpool2d": (lambda x: x.avgpool2d(pool_size=2, stride=2), [(2, 2, 6, 6)], ATOL),
    "composite": (lambda x, w: ((x.matmul(w) * 0.5).relu() + 0.1).softmax(), [(4, 3), (3, 6)], ATOL),
}


@pytest.mark.parametrize("name", list(CASES))
def test_gradcheck(Node, name):
    build, shapes, atol = CASES[name]
    print("gradcheck", name, flush=True)
    gradcheck(Node, build, [clear_x(s) for s in shapes], atol)


def leaf10(Node):
    return Node.leaf(np.arange(1, 11, dtype=np.float32), True)


@pytest.mark.parametrize("seed", [np.array([1.0], np.float32), np.ones(20, np.float32)])
def test_wrong_seed_length_rejected(Node, seed):
    x = leaf10(Node)
    z = x * 2
    with pytest.raises(ValueError):
        z.backward(seed)
    assert x.grad() is None and z.grad() is None  # nothing was touched
    z.release()
    x.release()


def test_c_level_seed_mismatch_is_a_noop(tlib, Node):
    x = leaf10(Node)
    z = x * 2
    s = np.ones(3, np.float32)
    tlib.ag_backward_from(z.ptr, s.ctypes.data_as(__import__("tinytorch_amd").F32P), 3)
    assert x.grad() is None
    z.release()
    x.release()


def test_none_seed_and_coercions(Node):
    x = leaf10(Node)
    z = x * 2
    z.backward(None)
    assert (z.grad() == 1.0).all() and (x.grad() == 2.0).all()
    z.release()
    x.release()
    for seed in (np.arange(1, 11, dtype=np.int32), np.arange(1, 11, dtype=np.float64),
                 np.arange(1, 21, dtype=np.float64)[::2]):
        x = leaf10(Node)
        z = x * 2
        z.backward(seed)
        assert (x.grad() == 2 * np.asarray(seed, np.float32)).all()
        z.release()
        x.release()


def test_deep_chain_1000(Node):
    v = Node.leaf(np.array([1.0, 2.0], np.float32), True)
    nodes, cur = [v], v
    for _ in range(1000):
        cur = cur + 1.0
        nodes.append(cur)
    cur.backward(None)
    assert np.allclose(v.grad(), 1.0)
    for n in nodes:
        n.release()


def test_shared_subgraph_accumulates_3x(Node):
    x = Node.leaf(np.array([1.0, 2.0, 3.0], np.float32), True)
    y = x * x
    z = y + y
    z.backward(None)
    g1 = x.grad().copy()
    assert np.allclose(g1, [4.0, 8.0, 12.0])
    z.backward(None)
    assert np.allclose(x.grad(), 3 * g1)
    for n in (z, y, x):
        n.release()


def test_nan_inf_backward(Node):
    x = Node.leaf(np.array([np.nan, 1.0], np.float32), True)
    y = x * x
    y.backward(None)
    assert x.grad().shape == (2,)
    y.release()
    x.release()
    x = Node.leaf(np.array([np.inf, -np.inf], np.float32), True)
    r = x.relu()
    r.backward(None)
    assert np.isfinite(x.grad()).all()
    r.release()
    x.release()


def test_requires_grad_flags(Node, tlib):
    a = Node.leaf(np.ones((2, 3), np.float32), False)
    w = Node.leaf(np.ones((3, 4), np.float32), True)
    c = a.matmul(w)
    assert tlib.ag_requires_grad(a.ptr) == 0 and tlib.ag_requires_grad(c.ptr) == 1
    c.backward(None)
    assert a.grad() is None and np.all(w.grad() == 2.0)
    for n in (c, w, a):
        n.release()


def rel(a, b):
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def test_rules_vs_oracle_larger(Node):
    """matmul / conv / pool / relu / padones / softmax backward at moderate
    shapes against the oracle's backward functions (rel err <= 1e-4)."""
    A = rng.uniform(-1, 1, (96, 130)).astype(np.float32)
    B = rng.uniform(-1, 1, (130, 70)).astype(np.float32)
    G = rng.standard_normal((96, 70)).astype(np.float32)
    na, nb = Node.leaf(A), Node.leaf(B)
    nc = na.matmul(nb)
    nc.backward(G)
    assert rel(na.grad(), orc.matmul_nt(G, B)) <= 1e-4
    assert rel(nb.grad(), orc.matmul_tn(A, G)) <= 1e-4
    for n in (nc, na, nb):
        n.release()

    x = rng.standard_normal((4, 5, 12, 12)).astype(np.float32)
    w = rng.standard_normal((7, 5, 3, 3)).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    nx, nw, nb_ = Node.leaf(x), Node.leaf(w), Node.leaf(b)
    ny = nx.conv2d(nw, nb_, stride=2, pad=1)
    g = rng.standard_normal(ny.value().shape).astype(np.float32)
    ny.backward(g)
    dx, dw, db = orc.conv2d_bwd(x, w, g, 2, 2, 1, 1)
    assert rel(nx.grad(), dx) <= 1e-4 and rel(nw.grad(), dw) <= 1e-4 and rel(nb_.grad(), db) <= 1e-4
    for n in (ny, nx, nw, nb_):
        n.release()

    # relu -> 2x2 max pool: one fused backward when the relu feeds only the
    # pool (the first call), the two separate steps when the relu feeds two
    # pools or already holds a gradient (a second call accumulates, and the
    # relu's backward then sees the accumulated gradient, as in the reference)
    x = rng.integers(-2, 3, (3, 4, 9, 8)).astype(np.float32)
    g = rng.standard_normal((3, 4, 4, 4)).astype(np.float32)
    dr = orc.maxpool_bwd(orc.relu_fwd(x), g, 2, 2, 2, 2)
    nx = Node.leaf(x)
    nr = nx.relu()
    ny = nr.maxpool2d(pool_size=2, stride=2)
    ny.backward(g)
    assert np.array_equal(nr.grad(), dr) and np.array_equal(nx.grad(), orc.relu_bwd(x, dr))
    ny.backward(g)
    dx2 = orc.relu_bwd(x, dr) + orc.relu_bwd(x, dr + dr)
    assert np.array_equal(nr.grad(), dr + dr) and np.array_equal(nx.grad(), dx2)
    for n in (ny, nr, nx):
        n.release()
    nx = Node.leaf(x)
    nr = nx.relu()
    n1, n2 = nr.maxpool2d(pool_size=2, stride=2), nr.maxpool2d(pool_size=2, stride=2)
    ns = n1 + n2
    ns.backward(g)
    assert np.array_equal(nr.grad(), dr + dr) and np.array_equal(nx.grad(), orc.relu_bwd(x, dr + dr))
    for n in (ns, n1, n2, nr, nx):
        n.release()
    # the fused backward leaves the relu's own gradient unwritten until it is
    # asked for: a second pass before any read, a read of the pool's gradient
    # first, and a release without a read all keep the values above
    for order in ("twice_unread", "pool_first", "unread"):
        nx = Node.leaf(x)
        nr = nx.relu()
        ny = nr.maxpool2d(pool_size=2, stride=2)
        ny.backward(g)
        if order == "twice_unread":
            ny.backward(g)
            assert np.array_equal(nx.grad(), dx2) and np.array_equal(nr.grad(), dr + dr)
        elif order == "pool_first":
            assert np.array_equal(ny.grad(), g)
            assert np.array_equal(nr.grad(), dr) and np.array_equal(nx.grad(), orc.relu_bwd(x, dr))
        else:
            assert np.array_equal(nx.grad(), orc.relu_bwd(x, dr))
        for n in (ny, nr, nx) if order != "unread" else (nr, ny, nx):
            n.release()

    # relu -> padones: fused backward on the first call, two steps after
    x = rng.integers(-2, 3, (6, 7)).astype(np.float32)
    g = rng.standard_normal((6, 8)).astype(np.float32)
    dr = orc.padones_bwd(g)
    nx = Node.leaf(x)
    nr = nx.relu()
    ny = nr.padones()
    ny.backward(g)
    assert np.array_equal(nr.grad(), dr) and np.array_equal(nx.grad(), orc.relu_bwd(x, dr))
    ny.backward(g)
    dx2 = orc.relu_bwd(x, dr) + orc.relu_bwd(x, dr + dr)
    assert np.array_equal(nr.grad(), dr + dr) and np.array_equal(nx.grad(), dx2)
    for n in (ny, nr, nx):
        n.release()

    x = rng.integers(-2, 2, (3, 4, 9, 9)).astype(np.float32)
    nx = Node.leaf(x)
    acc = np.zeros_like(x)
    for p, s in ((2, 2), (3, 2)):  # the second backward accumulates into x.grad
        ny = nx.maxpool2d(pool_size=p, stride=s)
        g = rng.standard_normal(ny.value().shape).astype(np.float32)
        ny.backward(g)
        acc = orc.maxpool_bwd(x, g, p, p, s, s) if p == 2 else acc + orc.maxpool_bwd(x, g, p, p, s, s)
        assert np.array_equal(nx.grad(), acc)
        ny.release()
    nx.release()
