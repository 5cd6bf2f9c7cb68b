"""The C ABI's failure contract on the GPU backend.

Reference contract: every constructor / op returns NULL on bad arguments,
shape mismatch or out of memory and never aborts (reference
include/tensor.h:32, src/tensor.c:8-18); tt_sgemm_rowmajor returns -1 when
its buffers cannot be allocated (src/gemm.c:584-588); backward rules skip
silently when an allocation fails (src/autograd.c:44-63,308-316).

Out of memory is forced from the host: TT_FAIL_ALLOC_AFTER=n in a child's
environment, or the tth_fail_alloc_after(n) hook, makes every device
allocation after the next n fail.  A launch failure of the direct
convolution is forced with TT_FAIL_DIRECT_CONV=1 in a child process.  No
test makes a kernel fault.
"""
import ctypes
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import orc
from tinytorch_amd import F32P

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD_OOM = textwrap.dedent("""
    import ctypes, sys, numpy as np
    sys.path.insert(0, {root!r})
    import tinytorch_amd
    from tinytorch_amd import F32P
    tinytorch_amd.require_gpu()
    L = tinytorch_amd.lib()
    shp = (ctypes.c_long * 2)(4, 5)
    a = np.ones((4, 5), np.float32)
    out = []
    out.append(int(bool(L.tt_new(shp, 2))))
    out.append(int(bool(L.tt_fromdata(a.ctypes.data_as(F32P), shp, 2))))
    out.append(int(bool(L.ag_leaf(None, 1))))
    A = np.ones((8, 8), np.float32); C = np.full((8, 8), 7.0, np.float32)
    out.append(L.tt_sgemm_rowmajor(8, 8, 8, A.ctypes.data_as(F32P), A.ctypes.data_as(F32P),
                                   C.ctypes.data_as(F32P), 1))
    out.append(int(np.all(C == 7.0)))
    out.append(L.tth_last_error())
    print("res", *out, flush=True)
""")


def test_env_fail_alloc_returns_null_child():
    """TT_FAIL_ALLOC_AFTER=0: constructors return NULL, tt_sgemm_rowmajor -1
    with C untouched, the runtime records the out-of-memory error (-11)."""
    env = dict(os.environ, TT_FAIL_ALLOC_AFTER="0")
    print("child TT_FAIL_ALLOC_AFTER=0", flush=True)
    p = subprocess.run([sys.executable, "-c", CHILD_OOM.format(root=ROOT)], env=env,
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    res = [int(v) for v in p.stdout.split("res", 1)[1].split()]
    assert res == [0, 0, 0, -1, 1, -11], res


def _cnn_graph(L, T, lab_p, B, flat):
    """Build the small CNN step graph from the parameter tensors T; returns
    (nodes, leaves, loss) or (nodes, leaves, None) at the first NULL."""
    nodes = []

    def k(n):
        if n:
            nodes.append(n)
        return n
    X = k(L.ag_leaf(T["x"], 0))
    ws = [k(L.ag_leaf(T[n], 1)) for n in ("w1", "b1", "w2", "b2", "wfc")]
    if not X or not all(ws):
        return nodes, ws, None
    w1, b1, w2, b2, wfc = ws
    h = k(L.ag_conv2d(X, w1, b1, 1, 1, 1, 1))
    for op in (lambda h: L.ag_relu(h), lambda h: L.ag_maxpool2d(h, 2, 2, 2, 2),
               lambda h: L.ag_conv2d(h, w2, b2, 1, 1, 1, 1), lambda h: L.ag_relu(h),
               lambda h: L.ag_maxpool2d(h, 2, 2, 2, 2), lambda h: L.ag_reshape(h, flat, 2),
               lambda h: L.ag_padones(h), lambda h: L.ag_matmul(h, wfc),
               lambda h: L.ag_softmax_ce(h, lab_p, B)):
        if not h:
            return nodes, ws, None
        h = k(op(h))
    return nodes, ws, h


def _grads(L, leaves, sizes):
    out = []
    for n, size in zip(leaves, sizes):
        g = L.ag_grad(n)
        if not g:
            out.append(None)
            continue
        d = L.tt_data(g)
        assert d, "tt_data of a computed gradient"
        out.append(np.ctypeslib.as_array(d, shape=(size,)).copy())
    return out


def test_alloc_failure_sweep_cnn_step(tlib):
    """For every allocation of a small CNN training step in turn, make it and
    every later one fail: each op either returns a node or NULL, the step
    never aborts or faults, and every parameter gradient that backward
    produced equals the unfailed run's bit for bit (a rule whose allocation
    failed leaves its gradients absent, not partial)."""
    L = tlib
    B = 4
    x, y, P = orc.cnn_inputs(B=B, H=8, W=8, F1=4, F2=8, seed=21)
    arrs = dict(x=x, **P)
    T = {}
    for name, a in arrs.items():
        a = np.ascontiguousarray(a, np.float32)
        shp = (ctypes.c_long * a.ndim)(*a.shape)
        T[name] = L.tt_fromdata(a.ctypes.data_as(F32P), shp, a.ndim)
        assert T[name]
    sizes = [arrs[n].size for n in ("w1", "b1", "w2", "b2", "wfc")]
    lab = np.ascontiguousarray(y, np.int32)
    lab_p = lab.ctypes.data_as(ctypes.POINTER(ctypes.c_int))
    flat = (ctypes.c_long * 2)(B, P["wfc"].shape[0] - 1)

    def step(n_ok):
        if n_ok is not None:
            assert L.tth_fail_alloc_after(n_ok) == 0
        try:
            nodes, leaves, loss = _cnn_graph(L, T, lab_p, B, flat)
            if loss:
                L.ag_backward(loss)
        finally:
            L.tth_fail_alloc_after(-1)
        grads = _grads(L, leaves, sizes) if all(leaves) else None
        for nd in nodes:
            L.ag_release(nd)
        assert L.tth_sync() == 0
        return loss is not None, grads

    ok, want = step(None)
    assert ok and all(g is not None for g in want)
    complete = False
    for n in range(0, 400):
        print("alloc failure after", n, flush=True)
        fwd_ok, got = step(n)
        if got is None:
            continue
        for g, w in zip(got, want):
            if g is not None:
                assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), n
        if fwd_ok and all(g is not None for g in got):
            complete = True
            break
    assert complete, "the step needs more than 400 allocations"
    for t in T.values():
        L.tt_release(t)


CHILD_CONV = textwrap.dedent("""
    import sys, numpy as np
    sys.path.insert(0, {root!r}); sys.path.insert(0, {oracle!r})
    import orc, tinytorch_amd
    tinytorch_amd.require_gpu()
    from tinytorch_amd.torch_py import Node
    B = 8
    x, y, P = orc.cnn_inputs(B=B, H=16, W=16, F1=8, F2=16, seed=13)
    ref = orc.cnn_step(x, y, **P)
    X = Node.leaf(x, False)
    ws = {{k: Node.leaf(v) for k, v in P.items()}}
    h = X.conv2d(ws["w1"], ws["b1"], stride=1, pad=1).relu().maxpool2d(2, 2)
    h = h.conv2d(ws["w2"], ws["b2"], stride=1, pad=1).relu().maxpool2d(2, 2)
    logits = h.reshape((B, P["wfc"].shape[0] - 1)).padones().matmul(ws["wfc"])
    loss = logits.softmax_ce(y)
    loss.backward(None)
    err = np.abs(logits.value() - ref["logits"]).max() / np.abs(ref["logits"]).max()
    errs = [err]
    for k, r in (("w1", "dw1"), ("b1", "db1"), ("w2", "dw2"), ("b2", "db2"), ("wfc", "dwfc")):
        g = ws[k].grad()
        errs.append(np.abs(g - ref[r]).max() / max(np.abs(ref[r]).max(), 1e-30))
    print("errs", *errs, flush=True)
""")


def test_direct_conv_launch_failure_falls_back_child():
    """With every direct-convolution launch failing (deferred forward,
    fused conv+relu, dX), ag_conv2d's output and every gradient still come
    out right: the forward falls back to the implicit / im2col GEMM when the
    pending launch fails, the backward to its GEMM forms."""
    env = dict(os.environ, TT_FAIL_DIRECT_CONV="1")
    print("child TT_FAIL_DIRECT_CONV=1", flush=True)
    p = subprocess.run([sys.executable, "-c",
                        CHILD_CONV.format(root=ROOT, oracle=os.path.join(ROOT, "oracle"))],
                       env=env, capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    errs = [float(v) for v in p.stdout.split("errs", 1)[1].split()]
    assert max(errs) <= 1e-4, errs
