"""Implicit-GEMM convolution (im2col folded into the GEMM's operand loads)
against the oracle's conv2d forward / backward (reference
src/ops_spatial.c:71-127, src/autograd.c:456-553), at the GEMM bar
max|err| / (sqrt(K) * max|A| * max|B|) <= 1e-4 with K the summed length."""
import numpy as np
import pytest

import orc
from tinytorch_amd.hip import DevBuf, check

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(4242)
TOL = 1e-4

CASES = [  # (N, C, H, W, F, HH, WW, sh, sw, ph, pw)
    (2, 3, 7, 7, 4, 3, 3, 1, 1, 1, 1), (2, 3, 7, 7, 4, 3, 3, 2, 2, 0, 0),
    (3, 4, 9, 8, 5, 3, 2, 2, 1, 2, 1), (1, 1, 5, 5, 1, 1, 1, 1, 1, 0, 0),
    (2, 5, 6, 6, 3, 5, 5, 1, 1, 2, 2), (3, 6, 11, 5, 7, 3, 3, 1, 1, 0, 0),
    (2, 2, 9, 13, 3, 3, 5, 1, 1, 1, 2), (5, 7, 10, 10, 9, 4, 4, 2, 2, 1, 1),
    (2, 130, 6, 6, 5, 3, 3, 1, 1, 1, 1),    # Kc = 1170: k range split to fit the tap table
    (2, 8, 6, 6, 130, 3, 3, 1, 1, 1, 1),    # dX: K = F*9 = 1170
    (8, 3, 32, 32, 32, 3, 3, 1, 1, 1, 1), (16, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1),
    (128, 3, 32, 32, 32, 3, 3, 1, 1, 1, 1), (128, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1),  # config 4
]


def err(got, ref, K, amax, bmax):
    d = np.abs(got.astype(np.float64) - ref).max()
    return d / (np.sqrt(K) * amax * bmax)


@pytest.mark.parametrize("case", CASES)
def test_implicit_conv_vs_oracle(tlib, case):
    N, C, H, W, F, HH, WW, sh, sw, ph, pw = case
    Ho, Wo = orc.conv_out(H, W, HH, WW, sh, sw, ph, pw)
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float32)
    w = rng.uniform(-1, 1, (F, C, HH, WW)).astype(np.float32)
    b = rng.uniform(-1, 1, F).astype(np.float32)
    g = rng.standard_normal((N, F, Ho, Wo)).astype(np.float32)
    dx_, dw_, db_, dg_ = DevBuf.from_np(x), DevBuf.from_np(w), DevBuf.from_np(b), DevBuf.from_np(g)
    geo = (N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo)
    print("implicit conv", case, flush=True)

    out = DevBuf(N * F * Ho * Wo)
    check(tlib.tt_k_conv2d_fwd_implicit(dx_.ptr, dw_.ptr, db_.ptr, out.ptr, *geo), "fwd")
    ref = orc.conv2d_fwd(x, w, b, sh, sw, ph, pw)
    Kc = C * HH * WW
    assert err(out.to_np(ref.shape) - b[None, :, None, None], ref - b[None, :, None, None],
               Kc, 1.0, 1.0) <= TOL

    rdx, rdw, rdb = orc.conv2d_bwd(x, w, g, sh, sw, ph, pw)
    Ncol = N * Ho * Wo
    gmax = float(np.abs(g).max())
    dW, dB = DevBuf(w.size), DevBuf(F)
    check(tlib.tt_k_conv2d_dw_implicit(dg_.ptr, dx_.ptr, dW.ptr, dB.ptr, *geo), "dw+db")
    assert err(dW.to_np(w.shape), rdw, Ncol, gmax, 1.0) <= TOL
    assert err(dB.to_np((F,)), rdb, Ncol, gmax, 1.0) <= TOL
    dW2 = DevBuf(w.size)
    check(tlib.tt_k_conv2d_dw_implicit(dg_.ptr, dx_.ptr, dW2.ptr, None, *geo), "dw")
    assert np.array_equal(dW2.to_np(w.shape), dW.to_np(w.shape))

    dX = DevBuf(x.size)
    rc = tlib.tt_k_conv2d_dx_implicit(dg_.ptr, dw_.ptr, dX.ptr, *geo)
    if sh == 1 and sw == 1 and ph <= HH - 1 and pw <= WW - 1:
        check(rc, "dx")
        assert err(dX.to_np(x.shape), rdx, F * HH * WW, gmax, 1.0) <= TOL
    else:
        assert rc != 0  # not covered: the caller keeps the explicit dcol + col2im path
    for bf in (dx_, dw_, db_, dg_, out, dW, dB, dW2, dX):
        bf.free()


def test_implicit_conv_rejects_bad_args(tlib):
    geo = (2, 3, 7, 7, 4, 3, 3, 1, 1, 1, 1, 7, 7)
    assert tlib.tt_k_conv2d_fwd_implicit(None, None, None, None, *geo) != 0
    # Ho inconsistent with the transposed-convolution form
    buf = DevBuf(1024)
    bad = (2, 3, 7, 7, 4, 3, 3, 1, 1, 1, 1, 6, 7)
    assert tlib.tt_k_conv2d_dx_implicit(buf.ptr, buf.ptr, buf.ptr, *bad) != 0
    buf.free()


@pytest.mark.parametrize("case", [(4, 3, 9, 9, 5, 3, 3, 1, 1, 1, 1), (3, 4, 9, 8, 5, 3, 2, 2, 1, 2, 1),
                                  (128, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1)])
def test_autograd_conv_through_implicit_path(tlib, case):
    """ag_conv2d forward and backward (dX, dW, db) with the implicit forms
    forced (tth_conv_config(0)) against the oracle's conv backward; stride-2
    dX falls back to dcol + col2im inside the same call."""
    from tinytorch_amd.torch_py import Node
    N, C, H, W, F, HH, WW, sh, sw, ph, pw = case
    Ho, Wo = orc.conv_out(H, W, HH, WW, sh, sw, ph, pw)
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float32)
    w = rng.uniform(-1, 1, (F, C, HH, WW)).astype(np.float32)
    b = rng.uniform(-1, 1, F).astype(np.float32)
    g = rng.standard_normal((N, F, Ho, Wo)).astype(np.float32)
    tlib.tth_conv_config(0)
    prev = tlib.tth_conv_lds(0)  # the LDS-staged kernels would take these shapes first
    try:
        X, Wn, Bn = Node.leaf(x), Node.leaf(w), Node.leaf(b)
        out = X.conv2d(Wn, Bn, (sh, sw), (ph, pw))
        out.backward(g)
        ref = orc.conv2d_fwd(x, w, b, sh, sw, ph, pw)
        rdx, rdw, rdb = orc.conv2d_bwd(x, w, g, sh, sw, ph, pw)
        gmax = float(np.abs(g).max())
        assert err(out.value(), ref, C * HH * WW, 1.0, 1.0) <= TOL
        assert err(Wn.grad(), rdw, N * Ho * Wo, gmax, 1.0) <= TOL
        assert err(Bn.grad(), rdb, N * Ho * Wo, gmax, 1.0) <= TOL
        assert err(X.grad(), rdx, F * HH * WW, gmax, 1.0) <= TOL
        for n in (out, X, Wn, Bn):
            n.release()
    finally:
        tlib.tth_conv_config(-1)
        tlib.tth_conv_lds(prev)
