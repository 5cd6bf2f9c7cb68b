"""Whole training steps of the BASELINE configs on the GPU against the oracle
(which is bit-identical to the reference's CPU path): MLP (config 2) and
CNN (config 4) at full size -- logits, probabilities and every weight
gradient within max relative error 1e-4 (max|diff| / max|ref|).  Both the
reference harness pattern (softmax -> host CE seed -> ag_backward_from) and
the fused device softmax-CE node are checked, through ctypes and through the
pybind11 Node module."""
import os
import sys

import numpy as np
import pytest

import orc

pytestmark = pytest.mark.gpu
TOL = 1e-4


def rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.fixture(scope="module")
def Node(tlib):
    from tinytorch_amd.torch_py import Node as _Node
    return _Node


def mlp_graph(Node, x, Ws):
    X = Node.leaf(x, False)
    n = [Node.leaf(w) for w in Ws]
    h = X.padones().matmul(n[0]).relu().padones().matmul(n[1]).relu().padones()
    return X, n, h.matmul(n[2])


@pytest.mark.parametrize("fused", [False, True])
def test_mlp_step_config2(Node, fused):
    x, y, Ws = orc.mlp_inputs()  # B=256, 784->512->256->10, He-normal, zero bias rows
    ref = orc.mlp_step(x, y, *Ws)
    print("mlp step fused=", fused, flush=True)
    X, n, logits = mlp_graph(Node, x, Ws)
    if fused:
        loss = logits.softmax_ce(y)
        loss.backward(None)
        p = loss.probs()
        assert abs(float(loss.value()[0]) - ref["loss"]) <= 1e-5 * max(1.0, ref["loss"])
        extra = [loss]
    else:
        probs = logits.softmax()
        p = probs.value()
        onehot = np.eye(10, dtype=np.float32)[y]
        logits.backward((p - onehot) / np.float32(len(y)))
        extra = [probs]
    assert rel(logits.value(), ref["logits"]) <= TOL
    assert rel(p, ref["probs"]) <= TOL
    for i, k in enumerate(("dW1", "dW2", "dW3")):
        assert rel(n[i].grad(), ref[k]) <= TOL, k
    for node in extra + [logits, X] + n:
        node.release()


def cnn_graph(Node, x, P):
    X = Node.leaf(x, False)
    w1, b1, w2, b2, wfc = (Node.leaf(P[k]) for k in ("w1", "b1", "w2", "b2", "wfc"))
    h = X.conv2d(w1, b1, stride=1, pad=1).relu().maxpool2d(2, 2)
    h = h.conv2d(w2, b2, stride=1, pad=1).relu().maxpool2d(2, 2)
    B = x.shape[0]
    h = h.reshape((B, P["wfc"].shape[0] - 1)).padones()
    return X, (w1, b1, w2, b2, wfc), h.matmul(wfc)


@pytest.mark.parametrize("fused", [False, True])
def test_cnn_step_config4(Node, fused):
    x, y, P = orc.cnn_inputs()  # B=128, 3x32x32, conv32, conv64, FC 4096->10
    ref = orc.cnn_step(x, y, **P)
    print("cnn step fused=", fused, flush=True)
    X, ws, logits = cnn_graph(Node, x, P)
    if fused:
        loss = logits.softmax_ce(y)
        loss.backward(None)
        p = loss.probs()
        extra = [loss]
    else:
        probs = logits.softmax()
        p = probs.value()
        onehot = np.eye(10, dtype=np.float32)[y]
        logits.backward((p - onehot) / np.float32(len(y)))
        extra = [probs]
    assert rel(logits.value(), ref["logits"]) <= TOL
    assert rel(p, ref["probs"]) <= TOL
    for node, k in zip(ws, ("dw1", "db1", "dw2", "db2", "dwfc")):
        r = rel(node.grad(), ref[k])
        print(k, r, flush=True)
        assert r <= TOL, k
    for node in extra + [logits, X] + list(ws):
        node.release()


def test_sgd_step_on_device(Node):
    w = np.random.default_rng(3).standard_normal((5, 4)).astype(np.float32)
    g = np.random.default_rng(4).standard_normal((5, 4)).astype(np.float32)
    W = Node.leaf(w)
    X = Node.leaf(np.eye(5, dtype=np.float32), False)
    out = X.matmul(W)
    out.backward(g)
    assert np.allclose(W.grad(), g, atol=1e-6)
    W.sgd_step(0.1)
    assert np.allclose(W.value(), w - np.float32(0.1) * g, atol=1e-6)
    for n in (out, X, W):
        n.release()


def test_pybind_drop_in_smoke():
    """examples/train_mnist.py --smoke pattern through tinytorch_pybind."""
    import tinytorch_amd
    sys.path.insert(0, os.path.join(tinytorch_amd.ROOT, "build"))
    import tinytorch_pybind as tt
    assert tt.available()
    rng = np.random.default_rng(42)
    w1v = (rng.standard_normal((785, 64)) * np.sqrt(2.0 / 785)).astype(np.float32)
    w2v = (rng.standard_normal((65, 10)) * np.sqrt(2.0 / 65)).astype(np.float32)
    for _ in range(2):
        xr = rng.standard_normal((32, 784)).astype(np.float32)
        y = rng.integers(0, 10, 32)
        xp = np.concatenate([xr, np.ones((32, 1), np.float32)], axis=1)
        w1, w2 = tt.Node.leaf(w1v, True), tt.Node.leaf(w2v, True)
        h1 = tt.Node.leaf(xp, False).matmul(w1).relu()
        logits = h1.padones().matmul(w2)
        p = logits.softmax().value()
        onehot = np.eye(10, dtype=np.float32)[y]
        logits.backward((p - onehot) / 32.0)
        # the same step on the oracle path
        a1 = xp @ w1v
        h = orc.relu_fwd(a1)
        assert rel(p, orc.softmax_fwd(orc.padones_fwd(h) @ w2v)) <= 1e-4
        g1, g2 = w1.grad(), w2.grad()
        assert g1.shape == w1v.shape and g2.shape == w2v.shape and np.isfinite(g1).all()
        w1v -= 0.05 * g1
        w2v -= 0.05 * g2
    with pytest.raises(ValueError):
        tt.Node.leaf(np.ones((2, 3), np.float32)).matmul(tt.Node.leaf(np.ones((4, 5), np.float32)))
    n = tt.Node.leaf(np.ones(4, np.float32))
    with pytest.raises(ValueError):
        n.mulscalar(2.0).backward(np.ones(3, np.float32))
