"""Device optimizers (SGD-momentum, Adam) and device-resident parameters.

The GPU update must equal the oracle's restatement of the reference
harnesses' NumPy optimizers bit for bit (elementwise float32/float64
arithmetic, no reduction): reference tests/gate_mnist_mlp.py:121-124 and
tests/gate_cifar_cnn.py:81-98.  Gradients are injected exactly through
out = I @ W, whose weight gradient I^T @ seed is the seed itself."""
import ctypes
import os
import sys

import numpy as np
import pytest

import orc

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHAPES = [(5, 4), (7, 3), (64, 33)]


@pytest.fixture(scope="module")
def tp(tlib):
    from tinytorch_amd import torch_py
    return torch_py


@pytest.fixture(scope="module")
def pb(tlib):
    sys.path.insert(0, os.path.join(ROOT, "build"))
    try:
        import tinytorch_pybind
    finally:
        sys.path.pop(0)
    return tinytorch_pybind


def inject(Node, params, grads):
    """one graph per parameter: out = I @ W, backward(seed = g)"""
    extra = []
    for W, g in zip(params, grads):
        X = Node.leaf(np.eye(g.shape[0], dtype=np.float32), False)
        out = X.matmul(W)
        out.backward(g)
        extra += [X, out]
    return extra


def run_steps(Node, Optim, kind, steps, seed, release):
    rng = np.random.default_rng(seed)
    w0 = [rng.standard_normal(s).astype(np.float32) for s in SHAPES]
    persist = [Node.leaf(w) for w in w0]
    opt = Optim.sgd_momentum(0.1, 0.9) if kind == "momentum" else Optim.adam()
    ref_w = [w.copy() for w in w0]
    ref_m = [np.zeros_like(w) for w in w0]
    ref_v = [np.zeros_like(w) for w in w0]
    for t in range(1, steps + 1):
        grads = [rng.standard_normal(s).astype(np.float32) * np.float32(10.0 ** rng.integers(-4, 2))
                 for s in SHAPES]
        leaves = [p.detach() for p in persist]
        extra = inject(Node, leaves, grads)
        for l, g in zip(leaves, grads):
            assert np.array_equal(l.grad(), g)
        opt.step(leaves)
        if kind == "momentum":
            for w, v, g in zip(ref_w, ref_m, grads):
                orc.momentum_step(w, v, g, 0.1, 0.9)
        else:
            orc.adam_step(ref_w, grads, ref_m, ref_v, t)
        for i, (p, r) in enumerate(zip(persist, ref_w)):
            got = p.value()
            assert np.array_equal(got, r), (kind, t, i, float(np.abs(got - r).max()))
        release(extra + leaves)
    if kind == "adam":
        assert opt.t == steps
    release(persist)
    return opt


@pytest.mark.parametrize("kind", ["momentum", "adam"])
def test_optim_ctypes_bit_exact(tp, kind):
    def rel(ns):
        for n in ns:
            n.release()
    opt = run_steps(tp.Node, tp.Optim, kind, 5, 11, rel)
    opt.release()


@pytest.mark.parametrize("kind", ["momentum", "adam"])
def test_optim_pybind_bit_exact(pb, kind):
    run_steps(pb.Node, pb.Optim, kind, 5, 12, lambda ns: None)


def test_optim_many_params_and_errors(tp):
    """more parameters than one launch takes (16), a parameter without a
    gradient keeps its value and state, and a changed list is rejected"""
    rng = np.random.default_rng(5)
    n = 21
    w0 = [rng.standard_normal((3, 2 + i)).astype(np.float32) for i in range(n)]
    persist = [tp.Node.leaf(w) for w in w0]
    opt = tp.Optim.adam(lr=0.01)
    ref_w = [w.copy() for w in w0]
    ref_m = [np.zeros_like(w) for w in w0]
    ref_v = [np.zeros_like(w) for w in w0]
    for t in (1, 2):
        grads = [rng.standard_normal(w.shape).astype(np.float32) for w in w0]
        leaves = [p.detach() for p in persist]
        skip = 7  # no gradient reaches leaf 7
        extra = inject(tp.Node, [l for i, l in enumerate(leaves) if i != skip],
                       [g for i, g in enumerate(grads) if i != skip])
        opt.step(leaves)
        idx = [i for i in range(n) if i != skip]
        orc.adam_step([ref_w[i] for i in idx], [grads[i] for i in idx],
                      [ref_m[i] for i in idx], [ref_v[i] for i in idx], t, lr=0.01)
        for p, r in zip(persist, ref_w):
            assert np.array_equal(p.value(), r)
        with pytest.raises(ValueError):
            opt.step(leaves[:-1])
        for x in extra + leaves:
            x.release()
    bad = [tp.Node.leaf(np.zeros((3, 3), np.float32)) for _ in range(n)]
    with pytest.raises(ValueError):
        opt.step(bad)  # element counts differ from the bound slots
    for x in bad + persist:
        x.release()
    opt.release()
    with pytest.raises(ValueError):
        tp.Optim.adam(beta1=1.0)


def test_optim_kernel_limits(tlib):
    VP = ctypes.c_void_p
    arr = (VP * 17)()
    n = (ctypes.c_long * 17)()
    assert tlib.tt_k_adam_multi(arr, arr, arr, arr, n, 17, *([ctypes.c_float(0.5)] * 5),
                                ctypes.c_double(0.1)) != 0
    assert tlib.tt_k_momentum_multi(arr, arr, arr, n, 17, ctypes.c_float(0.1),
                                    ctypes.c_float(0.9)) != 0
    assert tlib.tt_k_momentum_multi(arr, arr, arr, n, 0, ctypes.c_float(0.1),
                                    ctypes.c_float(0.9)) == 0


def test_zero_copy_value_view(pb):
    w = np.random.default_rng(8).standard_normal((33, 17)).astype(np.float32)
    W = pb.Node.leaf(w)
    view = W.value(copy=False)
    assert np.array_equal(view, w) and not view.flags.owndata
    # the view keeps the tensor alive after the node is gone
    X = pb.Node.leaf(np.eye(33, dtype=np.float32), False)
    # writes through the view reach the device before the next op
    view[0, :] = 2.0
    out = X.matmul(W)
    assert np.array_equal(out.value()[0], np.full(17, 2.0, np.float32))
    # the mirror is refreshed in place by a later value()
    leaf = W.detach()
    out2 = X.matmul(leaf)
    out2.backward(np.ones((33, 17), np.float32))
    leaf.sgd_step(0.5)
    expect = view.copy() - np.float32(0.5)
    W.value()
    assert np.array_equal(view, expect)
    g = leaf.grad(copy=False)
    assert np.array_equal(g, np.ones((33, 17), np.float32))
    del W, leaf, out, out2, X
    assert np.array_equal(view, expect)


@pytest.mark.parametrize("kind", ["momentum", "adam"])
def test_cnn_training_steps_with_device_optimizer(tp, kind):
    """Config-4 CNN (B=128) trained 3 steps with device-resident weights, the
    fused softmax-CE and the device optimizer.  The updated weights equal the
    NumPy-rule optimizer fed with the GPU's gradients bit for bit, so both
    trajectories stay identical and every step's gradients are compared with
    the oracle's CNN step at the GPU's own weights, by the GEMM bar
    e = max|g - g_ref| / (sqrt(K) * max|dY| * max|X|) (K = terms summed per
    gradient element; dY, X the GEMM's operands):
      step 1: e <= 1e-4;
      later steps: e <= 1e-2.  The step is piecewise linear: a conv output
      within rounding of 0 can take the other side of the relu (or a
      near-tie the other maxpool argmax) on the GPU than in the oracle,
      which moves one upstream gradient term into or out of the sum, an
      error of up to 1/sqrt(K) of the scale (2.8e-3 for conv1, 5.5e-3 for
      conv2).  With 4.2 M conv1 outputs such a flip happens about once per
      few steps; the strict bar is held on the initial weights here and in
      the single-step tests."""
    x, y, P = orc.cnn_inputs()
    names = ("w1", "b1", "w2", "b2", "wfc")
    persist = [tp.Node.leaf(P[k]) for k in names]
    X = tp.Node.leaf(x, False)
    ref = [P[k].copy() for k in names]
    ref_m = [np.zeros_like(r) for r in ref]
    ref_v = [np.zeros_like(r) for r in ref]
    opt = tp.Optim.sgd_momentum(0.01, 0.9) if kind == "momentum" else tp.Optim.adam()
    B = x.shape[0]
    for t in range(1, 4):
        ws = [p.detach() for p in persist]
        c1 = X.conv2d(ws[0], ws[1], 1, 1)
        p1 = c1.relu().maxpool2d(2, 2)
        c2 = p1.conv2d(ws[2], ws[3], 1, 1)
        h = c2.relu().maxpool2d(2, 2)
        hp = h.reshape([B, ws[4].value().shape[0] - 1]).padones()
        logits = hp.matmul(ws[4])
        loss = logits.softmax_ce(y)
        loss.backward()
        grads = [w.grad() for w in ws]
        r = orc.cnn_step(x, y, *ref)
        d1, d2, dl = np.abs(c1.grad()).max(), np.abs(c2.grad()).max(), np.abs(logits.grad()).max()
        K1, K2 = B * 32 * 32, B * 16 * 16
        scale = dict(dw1=np.sqrt(K1) * d1 * np.abs(x).max(), db1=np.sqrt(K1) * d1,
                     dw2=np.sqrt(K2) * d2 * np.abs(p1.value()).max(), db2=np.sqrt(K2) * d2,
                     dwfc=np.sqrt(B) * dl * np.abs(hp.value()).max())
        for k, g in zip(("dw1", "db1", "dw2", "db2", "dwfc"), grads):
            d = float(np.abs(g.astype(np.float64) - r[k]).max() / scale[k])
            print(kind, t, k, d, flush=True)
            assert d <= (1e-4 if t == 1 else 1e-2), (kind, t, k, d)
        opt.step(ws)
        if kind == "momentum":
            for w, v, g in zip(ref, ref_m, grads):
                orc.momentum_step(w, v, g, 0.01, 0.9)
        else:
            orc.adam_step(ref, grads, ref_m, ref_v, t)
        for k, p, rw in zip(names, persist, ref):
            assert np.array_equal(p.value(), rw), (kind, t, k)
        for n in [loss, logits, hp, h, c2, p1, c1] + ws:
            n.release()
    for n in persist + [X]:
        n.release()
    opt.release()
