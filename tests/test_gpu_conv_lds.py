"""LDS-staged direct convolution (image rows in LDS, MFMA operands read
through im2col addressing) against the oracle's conv2d forward / backward
(reference src/ops_spatial.c:71-127, src/autograd.c:456-553), at the GEMM
bar max|err| / (sqrt(K) * max|A| * max|B|) <= 1e-4, K the summed length."""
import numpy as np
import pytest

import orc
from tinytorch_amd.hip import DevBuf, check

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(5151)
TOL = 1e-4

CASES = [  # (N, C, H, W, F, HH, WW, sh, sw, ph, pw)
    (2, 3, 7, 7, 4, 3, 3, 1, 1, 1, 1), (2, 3, 7, 7, 4, 3, 3, 2, 2, 0, 0),
    (3, 4, 9, 8, 5, 3, 2, 2, 1, 2, 1), (1, 1, 5, 5, 1, 1, 1, 1, 1, 0, 0),
    (2, 5, 6, 6, 3, 5, 5, 1, 1, 2, 2), (3, 6, 11, 5, 7, 3, 3, 1, 1, 0, 0),
    (2, 2, 9, 13, 3, 3, 5, 1, 1, 1, 2), (5, 7, 10, 10, 9, 4, 4, 2, 2, 1, 1),
    (2, 3, 33, 31, 33, 3, 3, 1, 1, 1, 1),   # F = 33: a second, mostly empty filter block
    (2, 16, 12, 12, 70, 3, 3, 1, 1, 1, 1),  # K = 144, F = 70
    (2, 64, 8, 8, 20, 3, 3, 1, 1, 1, 1),    # K = 576: one 16-filter block, 36 tap blocks
    (3, 3, 17, 19, 8, 3, 3, 3, 3, 1, 1),    # stride 3, pixel count not a multiple of 4
    (2, 4, 40, 40, 6, 3, 3, 1, 1, 0, 0),    # 38 x 38 output: chunks that straddle rows
    (2, 1, 70, 70, 4, 3, 3, 1, 1, 1, 1),    # wide rows (Wp > 64)
    (8, 3, 32, 32, 32, 3, 3, 1, 1, 1, 1), (16, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1),
    (128, 3, 32, 32, 32, 3, 3, 1, 1, 1, 1), (128, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1),  # config 4
]


def err(got, ref, K, amax, bmax):
    d = np.abs(got.astype(np.float64) - ref).max()
    return d / (np.sqrt(K) * amax * bmax)


def _inputs(case):
    N, C, H, W, F, HH, WW, sh, sw, ph, pw = case
    Ho, Wo = orc.conv_out(H, W, HH, WW, sh, sw, ph, pw)
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float32)
    w = rng.uniform(-1, 1, (F, C, HH, WW)).astype(np.float32)
    b = rng.uniform(-1, 1, F).astype(np.float32)
    g = rng.standard_normal((N, F, Ho, Wo)).astype(np.float32)
    return x, w, b, g, (N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo)


@pytest.mark.parametrize("case", CASES)
def test_lds_conv_vs_oracle(tlib, case):
    x, w, b, g, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    print("lds conv", case, flush=True)
    bits = tlib.tt_k_conv2d_lds_plan(*geo)
    assert bits & 3 == 3, f"plan {bits}"
    stride1 = sh == 1 and sw == 1 and ph <= HH - 1 and pw <= WW - 1
    assert bool(bits & 4) == stride1
    dx_, dw_, db_, dg_ = DevBuf.from_np(x), DevBuf.from_np(w), DevBuf.from_np(b), DevBuf.from_np(g)

    out = DevBuf(N * F * Ho * Wo)
    check(tlib.tt_k_conv2d_fwd_lds(dx_.ptr, dw_.ptr, db_.ptr, out.ptr, *geo), "fwd")
    ref = orc.conv2d_fwd(x, w, b, sh, sw, ph, pw)
    Kc = C * HH * WW
    bb = b[None, :, None, None]
    assert err(out.to_np(ref.shape) - bb, ref - bb, Kc, 1.0, 1.0) <= TOL
    out0 = DevBuf(N * F * Ho * Wo)  # no bias
    check(tlib.tt_k_conv2d_fwd_lds(dx_.ptr, dw_.ptr, None, out0.ptr, *geo), "fwd nobias")
    assert err(out0.to_np(ref.shape), ref - bb, Kc, 1.0, 1.0) <= TOL

    rdx, rdw, rdb = orc.conv2d_bwd(x, w, g, sh, sw, ph, pw)
    Ncol = N * Ho * Wo
    gmax = float(np.abs(g).max())
    dW, dB = DevBuf(w.size), DevBuf(F)
    check(tlib.tt_k_conv2d_dw_lds(dg_.ptr, dx_.ptr, dW.ptr, dB.ptr, *geo), "dw+db")
    assert err(dW.to_np(w.shape), rdw, Ncol, gmax, 1.0) <= TOL
    assert err(dB.to_np((F,)), rdb, Ncol, gmax, 1.0) <= TOL
    dW2 = DevBuf(w.size)
    check(tlib.tt_k_conv2d_dw_lds(dg_.ptr, dx_.ptr, dW2.ptr, None, *geo), "dw")
    assert np.array_equal(dW2.to_np(w.shape), dW.to_np(w.shape))  # deterministic

    dX = DevBuf(x.size)
    rc = tlib.tt_k_conv2d_dx_lds(dg_.ptr, dw_.ptr, dX.ptr, *geo)
    if stride1:
        check(rc, "dx")
        assert err(dX.to_np(x.shape), rdx, F * HH * WW, gmax, 1.0) <= TOL
    else:
        assert rc == -1  # not covered: nothing launched
    for bf in (dx_, dw_, db_, dg_, out, out0, dW, dB, dW2, dX):
        bf.free()


@pytest.mark.parametrize("case", [(2, 3, 12, 12, 5, 3, 3, 1, 1, 1, 1),
                                  (2, 9, 10, 10, 4, 3, 3, 1, 1, 1, 1)])
def test_lds_conv_nonfinite_stays_local(tlib, case):
    """An Inf in the input reaches only the outputs whose window holds it:
    padded taps (past K) read a zero plane, never an input value times 0."""
    x, w, b, g, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    x[1, C - 1, H // 2, W // 3] = np.inf
    g[0, F - 1, 0, Wo - 1] = -np.inf
    ref = orc.conv2d_fwd(x, w, b, sh, sw, ph, pw)
    rdx, _, _ = orc.conv2d_bwd(x, w, g, sh, sw, ph, pw)
    dx_, dw_, db_, dg_ = DevBuf.from_np(x), DevBuf.from_np(w), DevBuf.from_np(b), DevBuf.from_np(g)
    out, dX = DevBuf(ref.size), DevBuf(x.size)
    check(tlib.tt_k_conv2d_fwd_lds(dx_.ptr, dw_.ptr, db_.ptr, out.ptr, *geo), "fwd")
    check(tlib.tt_k_conv2d_dx_lds(dg_.ptr, dw_.ptr, dX.ptr, *geo), "dx")
    o, d = out.to_np(ref.shape), dX.to_np(x.shape)
    assert np.array_equal(np.isfinite(o), np.isfinite(ref))
    assert np.array_equal(np.isfinite(d), np.isfinite(rdx))
    m = np.isfinite(ref)
    assert np.abs(o[m] - ref[m]).max() <= TOL * np.sqrt(C * HH * WW) * 2
    m = np.isfinite(rdx)
    assert np.abs(d[m] - rdx[m]).max() <= TOL * np.sqrt(F * HH * WW) * 4 * np.abs(g[np.isfinite(g)]).max()
    for bf in (dx_, dw_, db_, dg_, out, dX):
        bf.free()


def test_lds_conv_rejects_uncovered(tlib):
    buf = DevBuf(1 << 16)
    geo = (2, 3, 7, 7, 4, 3, 3, 1, 1, 1, 1, 7, 7)
    assert tlib.tt_k_conv2d_fwd_lds(None, None, None, None, *geo) == -1
    bad = (2, 3, 7, 7, 4, 3, 3, 1, 1, 1, 1, 6, 7)   # Ho inconsistent with the geometry
    assert tlib.tt_k_conv2d_lds_plan(*bad) == 0
    assert tlib.tt_k_conv2d_fwd_lds(buf.ptr, buf.ptr, None, buf.ptr, *bad) == -1
    # a 1 x 4096 x 4 x 4 input with a 3x3 kernel: the staged slab does not fit
    big = (1, 4096, 4, 4, 8, 3, 3, 1, 1, 1, 1, 4, 4)
    assert tlib.tt_k_conv2d_lds_plan(*big) & 1 == 0
    assert tlib.tt_k_conv2d_fwd_lds(buf.ptr, buf.ptr, None, buf.ptr, *big) == -1
    prev = tlib.tth_conv_lds(0)
    try:
        assert tlib.tt_k_conv2d_lds_plan(*geo) == 0
    finally:
        tlib.tth_conv_lds(prev)
    buf.free()


@pytest.mark.parametrize("lds", [1, 0])
@pytest.mark.parametrize("case", [(4, 3, 9, 9, 5, 3, 3, 1, 1, 1, 1), (3, 4, 9, 8, 5, 3, 2, 2, 1, 2, 1),
                                  (128, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1)])
def test_autograd_conv_lds_on_off(tlib, case, lds):
    """ag_conv2d forward + backward (dX, dW, db) with the LDS kernels on (the
    default) and off (im2col + GEMM) against the oracle."""
    from tinytorch_amd.torch_py import Node
    x, w, b, g, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    prev = tlib.tth_conv_lds(lds)
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
        tlib.tth_conv_lds(prev)


def _random_cases(n=40, seed=777):
    """Seeded random shapes spread over the kernel variants: 3x3 and other
    kernels, strides 1-3, paddings 0..k-1, odd/even widths (16-byte and 4-byte
    staging), channel counts from 1 to 48 (dW tap-block variants up to
    K = 432), filter counts across block boundaries."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        HH = int(r.choice([1, 2, 3, 3, 3, 5]))
        WW = HH if r.random() < 0.8 else int(r.choice([1, 2, 3]))
        sh, sw = int(r.integers(1, 4)), int(r.integers(1, 3))
        ph, pw = int(r.integers(0, HH)), int(r.integers(0, WW))
        H, W = int(r.integers(max(HH, 3), 24)), int(r.integers(max(WW, 3), 24))
        C, F, N = int(r.integers(1, 49)), int(r.integers(1, 70)), int(r.integers(1, 5))
        Ho = (H + 2 * ph - HH) // sh + 1
        Wo = (W + 2 * pw - WW) // sw + 1
        if Ho <= 0 or Wo <= 0:
            continue
        out.append((N, C, H, W, F, HH, WW, sh, sw, ph, pw))
    return out


@pytest.mark.parametrize("case", _random_cases())
def test_lds_conv_random_shapes(tlib, case):
    """Every entry the plan reports as covered, against the oracle."""
    x, w, b, g, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    print("lds conv random", case, flush=True)
    bits = tlib.tt_k_conv2d_lds_plan(*geo)
    dx_, dw_, db_, dg_ = DevBuf.from_np(x), DevBuf.from_np(w), DevBuf.from_np(b), DevBuf.from_np(g)
    gmax = float(np.abs(g).max())
    if bits & 1:
        out = DevBuf(N * F * Ho * Wo)
        check(tlib.tt_k_conv2d_fwd_lds(dx_.ptr, dw_.ptr, db_.ptr, out.ptr, *geo), "fwd")
        ref = orc.conv2d_fwd(x, w, b, sh, sw, ph, pw)
        bb = b[None, :, None, None]
        assert err(out.to_np(ref.shape) - bb, ref - bb, C * HH * WW, 1.0, 1.0) <= TOL
        out.free()
    rdx, rdw, rdb = orc.conv2d_bwd(x, w, g, sh, sw, ph, pw)
    if bits & 2:
        dW, dB = DevBuf(w.size), DevBuf(F)
        check(tlib.tt_k_conv2d_dw_lds(dg_.ptr, dx_.ptr, dW.ptr, dB.ptr, *geo), "dw")
        assert err(dW.to_np(w.shape), rdw, N * Ho * Wo, gmax, 1.0) <= TOL
        assert err(dB.to_np((F,)), rdb, N * Ho * Wo, gmax, 1.0) <= TOL
        dW.free(); dB.free()
    if bits & 4:
        dX = DevBuf(x.size)
        check(tlib.tt_k_conv2d_dx_lds(dg_.ptr, dw_.ptr, dX.ptr, *geo), "dx")
        assert err(dX.to_np(x.shape), rdx, F * HH * WW, gmax, 1.0) <= TOL
        dX.free()
    for bf in (dx_, dw_, db_, dg_):
        bf.free()


def _bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("case", CASES)
def test_conv_relu_fused_kernel_bitexact(tlib, case):
    """tt_k_conv2d_relu_fwd_lds: both outputs bit for bit equal to the
    convolution alone followed by the relu kernel (reference
    src/ops_spatial.c:71-127 then src/ops.c:104-106), NaN and -0 included."""
    x, w, b, _, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    x.flat[:: max(1, x.size // 7)] = np.nan  # NaN outputs: the relu gives +0
    print("conv relu fused", case, flush=True)
    n_out = N * F * Ho * Wo
    dx_, dw_, db_ = DevBuf.from_np(x), DevBuf.from_np(w), DevBuf.from_np(b)
    for bias in (db_.ptr, None):
        o1, r1, o2, r2 = DevBuf(n_out), DevBuf(n_out), DevBuf(n_out), DevBuf(n_out)
        check(tlib.tt_k_conv2d_relu_fwd_lds(dx_.ptr, dw_.ptr, bias, o1.ptr, r1.ptr, *geo), "fused")
        check(tlib.tt_k_conv2d_fwd_lds(dx_.ptr, dw_.ptr, bias, o2.ptr, *geo), "conv")
        check(tlib.tt_k_relu_fwd(o2.ptr, r2.ptr, n_out), "relu")
        shp = (N, F, Ho, Wo)
        assert _bits_equal(o1.to_np(shp), o2.to_np(shp))
        assert _bits_equal(r1.to_np(shp), r2.to_np(shp))
    assert tlib.tt_k_conv2d_relu_fwd_lds(dx_.ptr, dw_.ptr, None, o1.ptr, o1.ptr, *geo) == -1


@pytest.mark.parametrize("case", CASES[-4:] + CASES[:3])
def test_autograd_conv_relu_deferred(tlib, case):
    """ag_conv2d followed by ag_relu (one fused launch) against the same graph
    with every convolution launched at once: values and gradients bit for bit
    equal.  Reading the convolution's value before the relu, releasing it
    before the relu, and a relu on another tensor in between all launch the
    pending convolution first."""
    from tinytorch_amd.torch_py import Node
    x, w, b, _, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    g = rng.standard_normal((N, F, Ho, Wo)).astype(np.float32)
    print("deferred conv relu", case, flush=True)

    def run(mode):
        X, Wn, Bn = Node.leaf(x), Node.leaf(w), Node.leaf(b)
        c = X.conv2d(Wn, Bn, (sh, sw), (ph, pw))
        if mode == "peek":
            cv = c.value()          # launches the pending convolution
        if mode == "other":
            o = Bn.relu()           # a relu of another node: flushes, then runs alone
            o.release()
        r = c.relu()
        vals = [c.value(), r.value()]
        if mode == "release":
            c.release()             # r keeps the convolution node alive
        r.backward(g)
        out = vals + [X.grad(), Wn.grad(), Bn.grad()]
        if mode == "peek":
            assert _bits_equal(cv, vals[0])
        for n in ([r, X, Wn, Bn] if mode == "release" else [r, c, X, Wn, Bn]):
            n.release()
        return out

    prev = tlib.tth_conv_relu_fuse(0)
    try:
        ref = run("plain")
    finally:
        tlib.tth_conv_relu_fuse(prev)
    assert tlib.tth_conv_relu_fuse(-1) == 1
    for mode in ("fused", "peek", "other", "release"):
        got = run(mode)
        for a, e in zip(got, ref):
            assert _bits_equal(a, e), mode


DWT_CASES = CASES + [
    (4, 8, 16, 16, 40, 5, 5, 1, 1, 2, 2),   # 5x5 taps, F = 40: two filter blocks
    (3, 5, 20, 24, 7, 3, 3, 2, 2, 1, 1),    # stride 2
    (2, 64, 8, 8, 20, 3, 3, 1, 1, 1, 1),    # K = 576: six tap groups
    (1, 2, 4, 4, 3, 1, 1, 1, 1, 0, 0),      # 1x1, a single unit
    (9, 16, 12, 12, 33, 3, 3, 1, 1, 1, 1),  # units not a multiple of the groups
]


@pytest.mark.parametrize("case", DWT_CASES)
def test_conv_dw_tiled_vs_oracle(tlib, case):
    """The tiled weight gradient (where it applies) and the per-image kernel,
    each against the oracle, each deterministic run to run."""
    x, w, b, g, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    if not tlib.tt_k_conv2d_lds_plan(*geo) & 2:
        pytest.skip("weight gradient not covered by the LDS kernels")
    rdx, rdw, rdb = orc.conv2d_bwd(x, w, g, sh, sw, ph, pw)
    dx_, dg_ = DevBuf.from_np(x), DevBuf.from_np(g)
    gmax = float(np.abs(g).max())
    prev = tlib.tth_conv_dwt(-1)
    try:
        for on in (1, 0):
            tlib.tth_conv_dwt(on)
            print("conv dw tiled", on, case, flush=True)
            outs = []
            for _ in range(2):
                dW, dB = DevBuf(w.size), DevBuf(F)
                check(tlib.tt_k_conv2d_dw_lds(dg_.ptr, dx_.ptr, dW.ptr, dB.ptr, *geo), "dw")
                outs.append((dW.to_np(w.shape), dB.to_np((F,))))
            assert err(outs[0][0], rdw, N * Ho * Wo, gmax, 1.0) <= TOL
            assert err(outs[0][1], rdb, N * Ho * Wo, gmax, 1.0) <= TOL
            assert _bits_equal(outs[0][0], outs[1][0]) and _bits_equal(outs[0][1], outs[1][1])
    finally:
        tlib.tth_conv_dwt(prev)


POOL_CASES = [
    (128, 3, 32, 32, 32, 3, 3, 1, 1, 1, 1), (128, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1),  # config 4
    (128, 4, 32, 32, 8, 3, 3, 1, 1, 1, 1),  # Wo = 32 pairs blocks: needs two blocks a wave (N >= 128)
    (4, 16, 8, 8, 40, 3, 3, 1, 1, 1, 1), (2, 4, 4, 4, 8, 3, 3, 1, 1, 1, 1),
    (3, 5, 16, 16, 33, 3, 3, 1, 1, 1, 1),
]


@pytest.mark.parametrize("case", POOL_CASES)
def test_conv_relu_pool_fused_kernel_bitexact(tlib, case):
    """tt_k_conv2d_relu_pool_fwd_lds: convolution, relu and 2x2 / stride-2
    max pool bit for bit equal to the convolution + relu kernel followed by
    the pool kernel, and the pool equal to the oracle's max pool of the relu
    (reference src/ops_spatial.c:129-164), NaN inputs included."""
    x, w, b, _, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    x.flat[:: max(1, x.size // 5)] = np.nan
    print("conv relu pool fused", case, flush=True)
    n_out, n_pool = N * F * Ho * Wo, N * F * (Ho // 2) * (Wo // 2)
    dx_, dw_, db_ = DevBuf.from_np(x), DevBuf.from_np(w), DevBuf.from_np(b)
    o1, r1, p1 = DevBuf(n_out), DevBuf(n_out), DevBuf(n_pool)
    o2, r2, p2 = DevBuf(n_out), DevBuf(n_out), DevBuf(n_pool)
    K1 = F * (Ho // 2) * (Wo // 2)
    c1, d1 = DevBuf(n_pool), DevBuf(N * (K1 + 1))
    codes = DevBuf(n_pool, np.uint8)
    check(tlib.tt_k_conv2d_relu_pool_fwd_lds(dx_.ptr, dw_.ptr, db_.ptr, o1.ptr, r1.ptr, p1.ptr,
                                             c1.ptr, d1.ptr, codes.ptr, *geo), "fused")
    check(tlib.tt_k_conv2d_relu_fwd_lds(dx_.ptr, dw_.ptr, db_.ptr, o2.ptr, r2.ptr, *geo), "conv")
    check(tlib.tt_k_maxpool_fwd(r2.ptr, p2.ptr, N, F, Ho, Wo, 2, 2, 2, 2, Ho // 2, Wo // 2), "pool")
    shp, pshp = (N, F, Ho, Wo), (N, F, Ho // 2, Wo // 2)
    assert _bits_equal(o1.to_np(shp), o2.to_np(shp))
    assert _bits_equal(r1.to_np(shp), r2.to_np(shp))
    pool = p1.to_np(pshp)
    assert _bits_equal(pool, p2.to_np(pshp))
    assert _bits_equal(pool, orc.maxpool_fwd(r1.to_np(shp), 2, 2, 2, 2))
    flat = pool.reshape(N, K1)
    assert _bits_equal(c1.to_np((N, K1)), flat)
    assert _bits_equal(d1.to_np((N, K1 + 1)), orc.padones_fwd(flat))
    # the windows' codes: first argmax (top-left, top-right, bottom-left,
    # bottom-right) in bits 0-1, relu > 0 of the four in bits 2-5
    r = r1.to_np(shp)
    win = np.stack([r[:, :, 0::2, 0::2], r[:, :, 0::2, 1::2], r[:, :, 1::2, 0::2],
                    r[:, :, 1::2, 1::2]])
    want = np.argmax(win, axis=0).astype(np.uint8)
    for k in range(4):
        want |= ((win[k] > 0).astype(np.uint8) << (2 + k))
    assert np.array_equal(codes.to_np(pshp), want)
    # the pool + relu backward from the codes: bit for bit the one from the
    # relu values (the convolution output's gradient)
    gp = np.random.default_rng(3).standard_normal(pshp).astype(np.float32)
    gp.flat[::7] = -0.0
    dg = DevBuf.from_np(gp)
    e1, e2 = DevBuf(n_out), DevBuf(n_out)
    check(tlib.tt_k_maxpool2x2_code_relu_bwd(codes.ptr, dg.ptr, e1.ptr, N, F, Ho, Wo, Ho // 2,
                                             Wo // 2), "code bwd")
    check(tlib.tt_k_maxpool2x2_relu_bwd(r1.ptr, dg.ptr, None, e2.ptr, N, F, Ho, Wo, Ho // 2,
                                        Wo // 2), "relu bwd")
    assert _bits_equal(e1.to_np(shp), e2.to_np(shp))
    # the weight gradient from the pool gradient and the codes: bit for bit
    # the one from the decoded output gradient
    dw1, db1, dw2, db2 = DevBuf(w.size), DevBuf(F), DevBuf(w.size), DevBuf(F)
    covered = tlib.tt_k_conv2d_dw_lds_pooled(None, None, None, None, None, *geo) == 0
    if covered:
        check(tlib.tt_k_conv2d_dw_lds_pooled(dg.ptr, codes.ptr, dx_.ptr, dw1.ptr, db1.ptr, *geo),
              "pooled dw")
        check(tlib.tt_k_conv2d_dw_lds(e1.ptr, dx_.ptr, dw2.ptr, db2.ptr, *geo), "dw")
        assert _bits_equal(dw1.to_np(w.shape), dw2.to_np(w.shape))
        assert _bits_equal(db1.to_np((F,)), db2.to_np((F,)))


@pytest.mark.parametrize("case", [(2, 3, 24, 24, 4, 3, 3, 1, 1, 1, 1),   # 32 % Wo != 0
                                  (2, 3, 7, 7, 4, 3, 3, 1, 1, 1, 1),     # odd Ho, Wo
                                  (2, 3, 8, 8, 4, 5, 5, 1, 1, 2, 2),     # not 3x3
                                  (8, 3, 32, 32, 32, 3, 3, 1, 1, 1, 1)])  # Wo = 32, one block a wave
def test_conv_relu_pool_fused_rejects(tlib, case):
    x, w, b, _, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    dx_, dw_ = DevBuf.from_np(x), DevBuf.from_np(w)
    o, r, p = DevBuf(N * F * Ho * Wo), DevBuf(N * F * Ho * Wo), DevBuf(N * F * Ho * Wo)
    assert tlib.tt_k_conv2d_relu_pool_fwd_lds(dx_.ptr, dw_.ptr, None, o.ptr, r.ptr, p.ptr,
                                              None, None, None, *geo) == -1


@pytest.mark.parametrize("case", [POOL_CASES[3], POOL_CASES[5], (2, 3, 24, 24, 4, 3, 3, 1, 1, 1, 1)])
def test_autograd_conv_relu_pool_deferred(tlib, case):
    """ag_conv2d, ag_relu, ag_maxpool2d(2x2) in one launch against the same
    graph with every launch made at once: values and gradients bit for bit
    equal.  Reading the relu's value first, or a 3x3 pool, launches the
    pending convolution + relu alone (the pool then runs by itself)."""
    from tinytorch_amd.torch_py import Node
    x, w, b, _, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    print("deferred conv relu pool", case, flush=True)

    def run(mode):
        X, Wn, Bn = Node.leaf(x, mode != "nograd"), Node.leaf(w), Node.leaf(b)
        c = X.conv2d(Wn, Bn, (sh, sw), (ph, pw))
        r = c.relu()
        if mode == "peek":
            rv = r.value()
        k = 3 if mode == "pool3" else 2
        m = r.maxpool2d(k, k)
        mv = m.value()
        gm = np.ascontiguousarray(np.cos(np.arange(mv.size, dtype=np.float32)).reshape(mv.shape))
        if mode == "late":
            # the relu output is first read after the backward (which then
            # took the pool backward from the convolution output)
            m.backward(gm)
            vals = [c.value(), r.value(), mv]
        else:
            vals = [c.value(), r.value(), mv]
            m.backward(gm)
        out = vals + [Wn.grad(), Bn.grad(), r.grad(), c.grad()]
        if mode != "nograd":
            out.append(X.grad())
        if mode == "peek":
            assert _bits_equal(rv, vals[1])
        for nd in (m, r, c, X, Wn, Bn):
            nd.release()
        return out

    for mode in ("fused", "peek", "pool3", "late", "nograd"):
        prev = tlib.tth_conv_relu_fuse(0)
        try:
            ref = run(mode)
        finally:
            tlib.tth_conv_relu_fuse(prev)
        got = run(mode)
        for a, e in zip(got, ref):
            assert _bits_equal(a, e), mode


@pytest.mark.parametrize("mode", ["fused", "peek_pool", "reshape3d", "no_padones", "x_nograd"])
def test_autograd_conv_pool_flatten_deferred(tlib, mode):
    """The classifier's input chain conv -> relu -> 2x2 pool -> reshape ->
    padones (config 4's second convolution) as one launch, against the same
    graph with every launch made at once: values and gradients bit for bit
    equal.  Reading the pool first, a reshape that is not a flattening to 2-D,
    or a reshape not followed by a padones run the pending chain without the
    later steps."""
    from tinytorch_amd.torch_py import Node
    case = (16, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1)
    x, w, b, _, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    K1 = F * (Ho // 2) * (Wo // 2)
    print("deferred conv pool flatten", mode, flush=True)

    def run():
        X, Wn, Bn = Node.leaf(x, mode != "x_nograd"), Node.leaf(w), Node.leaf(b)
        m_relu = X.conv2d(Wn, Bn, (sh, sw), (ph, pw)).relu()
        m = m_relu.maxpool2d(2, 2)
        if mode == "peek_pool":
            m.value()
        nodes = [m]
        shape = (N, F, 1, K1 // F) if mode == "reshape3d" else (N, K1)
        rs = m.reshape(shape)
        nodes.append(rs)
        if mode == "reshape3d":
            rs = rs.reshape((N, K1))
            nodes.append(rs)
        top = rs
        if mode != "no_padones":
            top = rs.padones()
            nodes.append(top)
        v = top.value()
        gt = np.ascontiguousarray(np.sin(np.arange(v.size, dtype=np.float32)).reshape(v.shape))
        top.backward(gt)
        out = [v, m.value(), Wn.grad(), Bn.grad()]
        if mode != "x_nograd":
            out.append(X.grad())
        if mode in ("fused", "x_nograd"):
            # read last: the relu output and its gradient, both still recipes
            out += [m_relu.value(), m_relu.grad()]
        for nd in nodes[::-1] + [X, Wn, Bn]:
            nd.release()
        return out

    prev = tlib.tth_conv_relu_fuse(0)
    try:
        ref = run()
    finally:
        tlib.tth_conv_relu_fuse(prev)
    got = run()
    for a, e in zip(got, ref):
        assert _bits_equal(a, e), mode


def test_relu_recipe_survives_host_write_of_its_input(tlib):
    """The fused conv + relu + pool forward leaves the relu output as a
    recipe of the convolution output; writing the convolution output through
    its host pointer runs the recipe first, so the relu output keeps the
    values of the original convolution."""
    import ctypes
    from tinytorch_amd.torch_py import Node
    case = POOL_CASES[3]
    x, w, b, _, geo = _inputs(case)
    N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo = geo
    X, Wn, Bn = Node.leaf(x, False), Node.leaf(w), Node.leaf(b)
    c = X.conv2d(Wn, Bn, (sh, sw), (ph, pw))
    r = c.relu()
    m = r.maxpool2d(2, 2)
    m.value()  # launches the fused chain: the relu output is not stored
    ct = tlib.ag_value(c.ptr)
    hp = tlib.tt_data(ct)
    assert hp
    n = N * F * Ho * Wo
    buf = np.ctypeslib.as_array(ctypes.cast(hp, ctypes.POINTER(ctypes.c_float)), shape=(n,))
    orig = buf.copy().reshape(N, F, Ho, Wo)
    buf[:] = -3.0
    assert _bits_equal(r.value(), orc.relu_fwd(orig))
    for nd in (m, r, c, X, Wn, Bn):
        nd.release()


@pytest.mark.parametrize("order", ["read_all", "drop_first"])
def test_deferred_weight_gradient_reductions(tlib, order):
    """Two convolutions' weight-gradient reductions are left pending by the
    backward pass and run together when the first gradient is read; a
    pending reduction whose gradients are released unread writes nothing.
    The gradients are the oracle's (within tolerance) and the same bits in
    either order."""
    from tinytorch_amd.torch_py import Node
    r = np.random.default_rng(31)
    x = r.uniform(-1, 1, (4, 16, 8, 8)).astype(np.float32)
    w1 = r.uniform(-0.3, 0.3, (40, 16, 3, 3)).astype(np.float32)
    b1 = r.uniform(-1, 1, 40).astype(np.float32)
    w2 = r.uniform(-0.3, 0.3, (24, 40, 3, 3)).astype(np.float32)
    b2 = r.uniform(-1, 1, 24).astype(np.float32)
    g = r.standard_normal((4, 24, 8, 8)).astype(np.float32)

    def run(drop_first):
        X = Node.leaf(x, False)
        W1, B1, W2, B2 = Node.leaf(w1), Node.leaf(b1), Node.leaf(w2), Node.leaf(b2)
        c1 = X.conv2d(W1, B1, (1, 1), (1, 1))
        c2 = c1.conv2d(W2, B2, (1, 1), (1, 1))
        c2.backward(g)
        out = {}
        if drop_first:
            for nd in (W1, B1, c2, c1):  # W1's and B1's gradients released unread
                nd.release()
            out["w2"], out["b2"] = W2.grad(), B2.grad()
            for nd in (X, W2, B2):
                nd.release()
        else:
            out["w2"], out["b2"] = W2.grad(), B2.grad()
            out["w1"], out["b1"] = W1.grad(), B1.grad()
            for nd in (c2, c1, X, W1, B1, W2, B2):
                nd.release()
        return out

    got = run(order == "drop_first")
    ref = run(False)
    for k in got:
        assert _bits_equal(got[k], ref[k]), k
    y1 = orc.conv2d_fwd(x, w1, b1, 1, 1, 1, 1)
    dx1, dw2, db2 = orc.conv2d_bwd(y1, w2, g, 1, 1, 1, 1)
    _, dw1, db1 = orc.conv2d_bwd(x, w1, dx1, 1, 1, 1, 1)
    for k, want in (("w2", dw2), ("b2", db2), ("w1", dw1), ("b1", db1)):
        if k in got:
            e = np.abs(got[k] - want).max() / max(np.abs(want).max(), 1e-30)
            assert e <= 1e-4, (k, e)


def test_sgd_step_runs_pending_reductions(tlib):
    """ag_sgd_step_many on weights whose gradients are pending reductions:
    the reductions and the step in one launch give the same weights and
    gradients, bit for bit, as reading the gradients first (which runs the
    reductions) and stepping the plain way; a leaf without a pending
    reduction (the second bias is given no gradient path change) rides along."""
    import ctypes
    from tinytorch_amd.torch_py import Node
    r = np.random.default_rng(41)
    x = r.uniform(-1, 1, (4, 16, 8, 8)).astype(np.float32)
    ps = [r.uniform(-0.3, 0.3, (40, 16, 3, 3)), r.uniform(-1, 1, 40),
          r.uniform(-0.3, 0.3, (24, 40, 3, 3)), r.uniform(-1, 1, 24),
          r.uniform(-1, 1, (4, 24, 8, 8))]
    ps = [p.astype(np.float32) for p in ps]
    g = r.standard_normal((4, 24, 8, 8)).astype(np.float32)

    def run(read_first):
        X = Node.leaf(x, False)
        P = [Node.leaf(p) for p in ps]
        c1 = X.conv2d(P[0], P[1], (1, 1), (1, 1))
        c2 = c1.conv2d(P[2], P[3], (1, 1), (1, 1))
        y = c2 * P[4]  # a leaf whose gradient is an ordinary tensor
        y.backward(g)
        if read_first:
            for p in P:
                p.grad()
        arr = (ctypes.c_void_p * 5)(*[p.ptr for p in P])
        assert tlib.ag_sgd_step_many(arr, 5, ctypes.c_float(0.1)) == 0
        out = [p.value() for p in P] + [p.grad() for p in P]
        for nd in [y, c2, c1, X] + P:
            nd.release()
        return out

    fused, plain = run(False), run(True)
    for a, b in zip(fused, plain):
        assert _bits_equal(a, b)


def test_sgd_step_more_pending_reductions_than_one_launch_takes(tlib):
    """Five convolutions, so five pending weight-gradient reductions at the
    SGD step: more than the fused reduce + step launch takes (four jobs).
    The step then runs the reductions in their own launch and steps the
    plain way; weights and gradients bit for bit those of reading every
    gradient first."""
    import ctypes
    from tinytorch_amd.torch_py import Node
    r = np.random.default_rng(43)
    chans = [16, 24, 16, 24, 16, 24]
    x = r.uniform(-1, 1, (4, chans[0], 8, 8)).astype(np.float32)
    ps = []
    for ci, co in zip(chans[:-1], chans[1:]):
        ps.append(r.uniform(-0.3, 0.3, (co, ci, 3, 3)).astype(np.float32))
        ps.append(r.uniform(-1, 1, co).astype(np.float32))
    g = r.standard_normal((4, chans[-1], 8, 8)).astype(np.float32)

    def run(read_first):
        X = Node.leaf(x, False)
        P = [Node.leaf(p) for p in ps]
        hs = [X]
        for i in range(5):
            hs.append(hs[-1].conv2d(P[2 * i], P[2 * i + 1], (1, 1), (1, 1)))
        hs[-1].backward(g)
        if read_first:
            for p in P:
                p.grad()
        arr = (ctypes.c_void_p * len(P))(*[p.ptr for p in P])
        assert tlib.ag_sgd_step_many(arr, len(P), ctypes.c_float(0.05)) == 0
        out = [p.value() for p in P] + [p.grad() for p in P]
        for nd in hs[::-1] + P:
            nd.release()
        return out

    print("sgd step with five pending conv reductions", flush=True)
    fused, plain = run(False), run(True)
    for a, b in zip(fused, plain):
        assert _bits_equal(a, b)
