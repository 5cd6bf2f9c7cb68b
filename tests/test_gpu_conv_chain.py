"""The CNN feature extractor's two convolutions in one launch
(tt_k_conv2d_chain_fwd): conv -> relu -> 2x2 pool -> conv -> relu -> 2x2
pool must give, bit for bit, what two tt_k_conv2d_relu_pool_fwd_lds launches
give (convolution outputs, pools, the windows' codes, the flattened and
padded copies), and those are pinned against the oracle (reference
src/ops_spatial.c:71-164 with the relu of src/ops.c:104-106)."""
import numpy as np
import pytest

import orc
from tinytorch_amd.hip import DevBuf, check

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def geo(N, C, H, F):
    return (N, C, H, H, F, 3, 3, 1, 1, 1, 1, H, H)


# (N, C1, bias, nan): the config-4 batch, every channel count the kernel
# takes (one or two channel steps a lane half), no biases, NaN inputs
CASES = [(128, 3, True, False), (5, 1, True, False), (3, 2, False, False), (4, 4, True, True),
         (1, 3, True, False)]


@pytest.mark.parametrize("N,C1,bias,nan", CASES)
def test_conv_chain_matches_two_launches(tlib, N, C1, bias, nan):
    r = np.random.default_rng(100 + N + C1)
    x = r.uniform(0, 1, (N, C1, 32, 32)).astype(np.float32)
    if nan:
        x.flat[::97] = np.nan
    w1 = (r.standard_normal((32, C1, 3, 3)) * np.sqrt(2.0 / (9 * C1))).astype(np.float32)
    w2 = (r.standard_normal((64, 32, 3, 3)) * np.sqrt(2.0 / 288)).astype(np.float32)
    b1 = r.standard_normal(32).astype(np.float32) * 0.1 if bias else None
    b2 = r.standard_normal(64).astype(np.float32) * 0.1 if bias else None
    dx, dw1, dw2 = DevBuf.from_np(x), DevBuf.from_np(w1), DevBuf.from_np(w2)
    db1 = DevBuf.from_np(b1) if bias else None
    db2 = DevBuf.from_np(b2) if bias else None
    bp1, bp2 = (db1.ptr if bias else None), (db2.ptr if bias else None)
    n1, p1n, n2, p2n = N * 32 * 1024, N * 32 * 256, N * 64 * 256, N * 64 * 64
    print("conv chain", N, C1, bias, nan, flush=True)
    # the separate kernels: convolution + relu, max pool; codes from the relu
    # values (first argmax in top-left, top-right, bottom-left, bottom-right
    # order in bits 0-1, relu > 0 of the four in bits 2-5)
    o1, r1, p1 = DevBuf(n1), DevBuf(n1), DevBuf(p1n)
    o2, r2, p2 = DevBuf(n2), DevBuf(n2), DevBuf(p2n)
    check(tlib.tt_k_conv2d_relu_fwd_lds(dx.ptr, dw1.ptr, bp1, o1.ptr, r1.ptr, *geo(N, C1, 32, 32)),
          "conv1")
    check(tlib.tt_k_maxpool_fwd(r1.ptr, p1.ptr, N, 32, 32, 32, 2, 2, 2, 2, 16, 16), "pool1")
    check(tlib.tt_k_conv2d_relu_fwd_lds(p1.ptr, dw2.ptr, bp2, o2.ptr, r2.ptr, *geo(N, 32, 16, 64)),
          "conv2")
    check(tlib.tt_k_maxpool_fwd(r2.ptr, p2.ptr, N, 64, 16, 16, 2, 2, 2, 2, 8, 8), "pool2")

    def codes(r):
        win = np.stack([r[:, :, 0::2, 0::2], r[:, :, 0::2, 1::2], r[:, :, 1::2, 0::2],
                        r[:, :, 1::2, 1::2]])
        want = np.argmax(win, axis=0).astype(np.uint8)
        for k in range(4):
            want |= ((win[k] > 0).astype(np.uint8) << (2 + k))
        return want

    k1 = codes(r1.to_np((N, 32, 32, 32)))
    k2 = codes(r2.to_np((N, 64, 16, 16)))
    flat = p2.to_np((N, 4096))
    # one launch
    s1, j1 = DevBuf(p1n), DevBuf(p1n, np.uint8)
    s2, e2, f2, j2 = DevBuf(p2n), DevBuf(p2n), DevBuf(N * 4097), DevBuf(p2n, np.uint8)
    K1 = C1 * 9
    sa, sb = DevBuf(32 * K1 + 32), DevBuf(18432 + 64)
    # and a 10-class classifier's partial logits over each image half
    fcw = (r.standard_normal((4096, 10)) / 64.0).astype(np.float32)
    dfcw, fcp = DevBuf.from_np(fcw), DevBuf(2 * N * 10)
    check(tlib.tt_k_conv2d_chain_fwd(dx.ptr, dw1.ptr, bp1, dw2.ptr, bp2, s1.ptr, j1.ptr, s2.ptr,
                                     e2.ptr, f2.ptr, j2.ptr, sa.ptr, sb.ptr, dfcw.ptr, 10, fcp.ptr,
                                     N, C1, 32, 32, 32, 64),
          "chain")
    part = fcp.to_np((2, N, 10))
    feat = flat.astype(np.float64).reshape(N, 64, 64)
    for h in range(2):
        fh = feat[:, :, 32 * h:32 * h + 32].reshape(N, 2048)
        wh = fcw.astype(np.float64).reshape(64, 64, 10)[:, 32 * h:32 * h + 32].reshape(2048, 10)
        ref = fh @ wh
        bar = 1e-4 * np.sqrt(2048) * max(1e-30, np.abs(fh).max() * np.abs(wh).max())
        assert np.abs(part[h] - ref).max() <= bar
    assert bits_equal(p1.to_np((N, 32, 16, 16)), s1.to_np((N, 32, 16, 16)))
    assert bits_equal(p2.to_np((N, 64, 8, 8)), s2.to_np((N, 64, 8, 8)))
    assert bits_equal(e2.to_np((N, 4096)), flat)
    assert bits_equal(f2.to_np((N, 4097)), orc.padones_fwd(flat))
    assert bits_equal(j1.to_np((N, 32, 16, 16)), k1)
    assert bits_equal(j2.to_np((N, 64, 8, 8)), k2)
    zb1 = b1 if bias else np.zeros(32, np.float32)
    zb2 = b2 if bias else np.zeros(64, np.float32)
    assert bits_equal(sa.to_np((sa.n,)), np.concatenate([w1.ravel(), zb1]))
    assert bits_equal(sb.to_np((sb.n,)), np.concatenate([w2.ravel(), zb2]))
    # the convolution outputs recomputed from the snapshots: the same bits
    y1, y2 = DevBuf(n1), DevBuf(n2)
    check(tlib.tt_k_conv2d_fwd_lds(dx.ptr, sa.ptr, sa.ptr + 4 * 32 * K1, y1.ptr, *geo(N, C1, 32, 32)),
          "recompute 1")
    check(tlib.tt_k_conv2d_fwd_lds(s1.ptr, sb.ptr, sb.ptr + 4 * 18432, y2.ptr, *geo(N, 32, 16, 64)),
          "recompute 2")
    assert bits_equal(y1.to_np((N, 32, 32, 32)), o1.to_np((N, 32, 32, 32)))
    assert bits_equal(y2.to_np((N, 64, 16, 16)), o2.to_np((N, 64, 16, 16)))
    # optional outputs left out: the rest unchanged
    s1b, j1b, s2b, j2b = DevBuf(p1n), DevBuf(p1n, np.uint8), DevBuf(p2n), DevBuf(p2n, np.uint8)
    check(tlib.tt_k_conv2d_chain_fwd(dx.ptr, dw1.ptr, bp1, dw2.ptr, bp2, s1b.ptr, j1b.ptr, s2b.ptr,
                                     None, None, j2b.ptr, None, None, None, 0, None, N, C1, 32, 32,
                                     32, 64),
          "chain, pools only")
    assert bits_equal(s1b.to_np((N, 32, 16, 16)), s1.to_np((N, 32, 16, 16)))
    assert bits_equal(s2b.to_np((N, 64, 8, 8)), s2.to_np((N, 64, 8, 8)))
    assert bits_equal(j1b.to_np((N, 32, 16, 16)), j1.to_np((N, 32, 16, 16)))
    assert bits_equal(j2b.to_np((N, 64, 8, 8)), j2.to_np((N, 64, 8, 8)))
    if nan or N > 8:
        return
    # against the oracle: each convolution within the fp32 bar, each pool the
    # max pool of the relu of the GPU's own convolution output, bit for bit
    b1z = b1 if bias else np.zeros(32, np.float32)
    b2z = b2 if bias else np.zeros(64, np.float32)
    y1 = o1.to_np((N, 32, 32, 32))
    ref1 = orc.conv2d_fwd(x, w1, b1z, 1, 1, 1, 1)
    assert np.abs(y1 - ref1).max() <= 1e-4 * max(1.0, np.abs(ref1).max())
    assert bits_equal(s1.to_np((N, 32, 16, 16)), orc.maxpool_fwd(orc.relu_fwd(y1), 2, 2, 2, 2))
    pool1 = s1.to_np((N, 32, 16, 16))
    y2 = o2.to_np((N, 64, 16, 16))
    ref2 = orc.conv2d_fwd(pool1, w2, b2z, 1, 1, 1, 1)
    assert np.abs(y2 - ref2).max() <= 1e-4 * max(1.0, np.abs(ref2).max())
    assert bits_equal(s2.to_np((N, 64, 8, 8)), orc.maxpool_fwd(orc.relu_fwd(y2), 2, 2, 2, 2))


def test_conv_chain_rejects(tlib):
    d = DevBuf(64)
    assert tlib.tt_k_conv2d_chain_fwd(d.ptr, d.ptr, None, d.ptr, None, d.ptr, d.ptr, d.ptr, None,
                                      None, d.ptr, None, None, None, 0, None, 2, 5, 32, 32, 32,
                                      64) == -1
    assert tlib.tt_k_conv2d_chain_fwd(d.ptr, d.ptr, None, d.ptr, None, d.ptr, d.ptr, d.ptr, None,
                                      None, d.ptr, None, None, None, 0, None, 2, 3, 16, 16, 32,
                                      64) == -1


def _cnn(Node, x, P, keep):
    X = Node.leaf(x, False)
    w1, b1, w2, b2, wfc = (Node.leaf(P[k]) for k in ("w1", "b1", "w2", "b2", "wfc"))
    c1 = X.conv2d(w1, b1, stride=1, pad=1)
    r1 = c1.relu()
    p1 = r1.maxpool2d(2, 2)
    c2 = p1.conv2d(w2, b2, stride=1, pad=1)
    r2 = c2.relu()
    p2 = r2.maxpool2d(2, 2)
    f = p2.reshape((x.shape[0], P["wfc"].shape[0] - 1))
    d = f.padones()
    logits = d.matmul(wfc)
    keep.extend([X, w1, b1, w2, b2, wfc, c1, r1, p1, c2, r2, p2, f, d, logits])
    return logits


@pytest.mark.parametrize("B,read_early", [(16, False), (16, True), (128, False), (128, True)])
def test_autograd_chain_on_off_bitexact(tlib, B, read_early):
    """The config-4 graph through ag_*: with the two-convolution chain
    (one launch, convolution outputs recomputed from the filter snapshot on
    first read, the classifier's partial sums from the same launch) every
    value up to the classifier is bit for bit the graph without it and the
    rest within the fp32 bar,
    also when the convolution and relu outputs are read after an SGD step has
    changed the filters in place (the recipes read the snapshot), and when
    read before the backward pass.  At B = 128 the backward also takes the
    one-launch middle (the second convolution's input gradient and the first
    one's weight gradient: tt_k_conv2d_chain_bwd)."""
    from tinytorch_amd.torch_py import Node
    x, y, P = orc.cnn_inputs(B=B)
    names = ("X", "w1", "b1", "w2", "b2", "wfc", "c1", "r1", "p1", "c2", "r2", "p2", "f", "d",
             "logits")

    def run(chain):
        prev = tlib.tth_conv_chain(1 if chain else 0)
        keep = []
        try:
            logits = _cnn(Node, x, P, keep)
            loss = logits.softmax_ce(y)
            vals = {}
            if read_early:
                for k in ("c1", "r1", "c2", "r2"):
                    vals[k + "_early"] = keep[names.index(k)].value()
            loss.backward(None)
            grads = {k: keep[names.index(k)].grad()
                     for k in ("w1", "b1", "w2", "b2", "wfc", "d", "f", "p2", "c2")}
            for k in ("w1", "b1", "w2", "b2", "wfc"):
                keep[names.index(k)].sgd_step(0.5)
            for k, nd in zip(names, keep):
                vals[k] = nd.value()
            vals["loss"] = loss.value()
            for nd in [loss] + keep[::-1]:
                nd.release()
            return vals, grads
        finally:
            tlib.tth_conv_chain(prev)

    print("autograd chain on/off, B", B, "read_early", read_early, flush=True)
    (v1, g1), (v0, g0) = run(True), run(False)
    # everything up to the classifier bit for bit; the classifier's logits
    # come from the chain's two partial sums per image instead of the split-K
    # GEMM's, so they, the loss, the gradients and the stepped weights agree
    # to the fp32 bar (max |diff| <= 1e-4 max |value|)
    exact = ("X", "c1", "r1", "p1", "c2", "r2", "p2", "f", "d", "c1_early", "r1_early",
             "c2_early", "r2_early")
    for k in v0:
        if k in exact:
            assert bits_equal(v1[k], v0[k]), k
        else:
            assert np.abs(v1[k] - v0[k]).max() <= 1e-4 * max(1e-30, np.abs(v0[k]).max()), k
    for k in g0:
        assert np.abs(g1[k] - g0[k]).max() <= 1e-4 * max(1e-30, np.abs(g0[k]).max()), k
    # the recomputed convolution is the one of the filters before the step
    ref = orc.conv2d_fwd(x[:8], P["w1"], P["b1"], 1, 1, 1, 1)
    assert np.abs(v1["c1"][:8] - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())


def test_autograd_chain_second_conv_not_pooled(tlib):
    """conv -> relu -> pool -> conv -> relu with no second pool: the first
    convolution is launched by itself when the chain cannot complete, the
    values bit for bit those without the chain."""
    from tinytorch_amd.torch_py import Node
    x, y, P = orc.cnn_inputs(B=4)

    def run(chain):
        prev = tlib.tth_conv_chain(1 if chain else 0)
        try:
            X = Node.leaf(x, False)
            w1, b1, w2, b2 = (Node.leaf(P[k]) for k in ("w1", "b1", "w2", "b2"))
            c1 = X.conv2d(w1, b1, stride=1, pad=1)
            r1 = c1.relu()
            p1 = r1.maxpool2d(2, 2)
            c2 = p1.conv2d(w2, b2, stride=1, pad=1)
            r2 = c2.relu()
            out = [r2.value(), p1.value(), c1.value()]
            g = np.ones_like(out[0])
            r2.backward(g)
            out += [w1.grad(), w2.grad()]
            for nd in (r2, c2, p1, r1, c1, X, w1, b1, w2, b2):
                nd.release()
            return out
        finally:
            tlib.tth_conv_chain(prev)

    for a, b in zip(run(True), run(False)):
        assert bits_equal(a, b)


# (N, C1): the config-4 batch, other channel counts; the kernel covers the
# batches whose pooled weight gradient takes units of 8 rows (128 <= N < 256),
# the others return -1 (the separate kernels run instead)
BWD_CASES = [(128, 3), (130, 1), (200, 2), (5, 3), (256, 3)]


@pytest.mark.parametrize("N,C1", BWD_CASES)
def test_conv_chain_bwd_matches_separate(tlib, N, C1):
    """tt_k_conv2d_chain_bwd: dx2 bit for bit tt_k_conv2d_dx_lds, and dw1 /
    db1 bit for bit tt_k_conv2d_dw_lds_pooled of that dx2 with the pool
    codes; dx2 and dw1 within the bar of the oracle's conv backward and
    pool + relu backward (reference src/autograd.c:456-594)."""
    r = np.random.default_rng(200 + N + C1)
    x = r.uniform(0, 1, (N, C1, 32, 32)).astype(np.float32)
    w1 = (r.standard_normal((32, C1, 3, 3)) * np.sqrt(2.0 / (9 * C1))).astype(np.float32)
    b1 = (r.standard_normal(32) * 0.1).astype(np.float32)
    w2 = (r.standard_normal((64, 32, 3, 3)) * np.sqrt(2.0 / 288)).astype(np.float32)
    g = r.standard_normal((N, 64, 16, 16)).astype(np.float32)
    g.flat[::11] = 0.0
    dx, dw1_, db1_, dw2_, dg = (DevBuf.from_np(a) for a in (x, w1, b1, w2, g))
    # the first pool's codes and output from the forward kernels
    o1, p1 = DevBuf(N * 32 * 1024), DevBuf(N * 32 * 256)
    codes = DevBuf(N * 32 * 256, np.uint8)
    r1 = DevBuf(N * 32 * 1024)
    check(tlib.tt_k_conv2d_relu_fwd_lds(dx.ptr, dw1_.ptr, db1_.ptr, o1.ptr, r1.ptr,
                                        *geo(N, C1, 32, 32)), "conv1")
    rv = r1.to_np((N, 32, 32, 32))
    win = np.stack([rv[:, :, 0::2, 0::2], rv[:, :, 0::2, 1::2], rv[:, :, 1::2, 0::2],
                    rv[:, :, 1::2, 1::2]])
    cv = np.argmax(win, axis=0).astype(np.uint8)
    for k in range(4):
        cv |= ((win[k] > 0).astype(np.uint8) << (2 + k))
    codes = DevBuf.from_np(cv)
    print("conv chain bwd", N, C1, flush=True)
    # separate kernels
    ex, ew, eb = DevBuf(N * 32 * 256), DevBuf(w1.size), DevBuf(32)
    check(tlib.tt_k_conv2d_dx_lds(dg.ptr, dw2_.ptr, ex.ptr, *geo(N, 32, 16, 64)), "dx2")
    check(tlib.tt_k_conv2d_dw_lds_pooled(ex.ptr, codes.ptr, dx.ptr, ew.ptr, eb.ptr,
                                         *geo(N, C1, 32, 32)), "dw1 pooled")
    # one launch
    fx, fw, fb = DevBuf(N * 32 * 256), DevBuf(w1.size), DevBuf(32)
    rc = tlib.tt_k_conv2d_chain_bwd(dg.ptr, dw2_.ptr, codes.ptr, dx.ptr, fx.ptr, fw.ptr, fb.ptr,
                                    None, None, None, N, C1)
    if not 128 <= N < 256:
        assert rc == -1
        return
    check(rc, "chain bwd")
    assert bits_equal(fx.to_np((N, 32, 16, 16)), ex.to_np((N, 32, 16, 16)))
    assert bits_equal(fw.to_np(w1.shape), ew.to_np(w1.shape))
    assert bits_equal(fb.to_np((32,)), eb.to_np((32,)))
    # with the second convolution's weight gradient in the same grid: bit for
    # bit tt_k_conv2d_dw_lds of dc2 and the pool (its input)
    p1 = DevBuf.from_np(orc.maxpool_fwd(rv, 2, 2, 2, 2))
    e2w, e2b = DevBuf(w2.size), DevBuf(64)
    check(tlib.tt_k_conv2d_dw_lds(dg.ptr, p1.ptr, e2w.ptr, e2b.ptr, *geo(N, 32, 16, 64)), "dw2")
    gx, gw, gb, g2w, g2b = DevBuf(N * 32 * 256), DevBuf(w1.size), DevBuf(32), DevBuf(w2.size), DevBuf(64)
    check(tlib.tt_k_conv2d_chain_bwd(dg.ptr, dw2_.ptr, codes.ptr, dx.ptr, gx.ptr, gw.ptr, gb.ptr,
                                     p1.ptr, g2w.ptr, g2b.ptr, N, C1), "chain bwd + dw2")
    assert bits_equal(gx.to_np((N, 32, 16, 16)), ex.to_np((N, 32, 16, 16)))
    assert bits_equal(gw.to_np(w1.shape), ew.to_np(w1.shape))
    assert bits_equal(gb.to_np((32,)), eb.to_np((32,)))
    assert bits_equal(g2w.to_np(w2.shape), e2w.to_np(w2.shape))
    assert bits_equal(g2b.to_np((64,)), e2b.to_np((64,)))
    if N != 130:
        return
    # oracle: dx2, then the pool + relu backward and conv1's dw / db
    pool1 = orc.maxpool_fwd(rv, 2, 2, 2, 2)
    rdx = orc.conv2d_bwd(pool1, w2, g, 1, 1, 1, 1, need_dw=False, need_db=False)[0]
    dx2 = fx.to_np((N, 32, 16, 16))
    assert np.abs(dx2 - rdx).max() <= 1e-4 * max(1.0, np.abs(rdx).max())
    gr = orc.relu_bwd(rv, orc.maxpool_bwd(rv, dx2, 2, 2, 2, 2))
    _, rdw, rdb = orc.conv2d_bwd(x, w1, gr, 1, 1, 1, 1, need_dx=False)
    assert np.abs(fw.to_np(w1.shape) - rdw).max() <= 1e-4 * max(1.0, np.abs(rdw).max())
    assert np.abs(fb.to_np((32,)) - rdb).max() <= 1e-4 * max(1.0, np.abs(rdb).max())


@pytest.mark.parametrize("when", ["before", "never", "after"])
def test_autograd_chain_softmax_ce_recipe(tlib, when):
    """The config-4 graph with the chain's classifier partial sums: the
    softmax-CE's outputs are formed by the classifier backward (when the
    backward runs first) or by their own reduction on a first read before
    it; read before, after, or never (the graph released unread, then a full
    step run again), the loss, probabilities and gradients match the graph
    without the chain to the fp32 bar and the oracle's loss."""
    from tinytorch_amd.torch_py import Node
    x, y, P = orc.cnn_inputs(B=128)
    ref = orc.cnn_step(x, y, **P)

    def run(chain, when):
        prev = tlib.tth_conv_chain(1 if chain else 0)
        keep = []
        try:
            logits = _cnn(Node, x, P, keep)
            loss = logits.softmax_ce(y)
            out = {}
            if when == "before":
                out["loss"] = loss.value()
                out["probs"] = loss.probs()
            if when != "never":
                loss.backward(None)
                out["dwfc"] = keep[5].grad()
                out["dw2"] = keep[3].grad()
                if when == "after":
                    out["loss"] = loss.value()
                    out["probs"] = loss.probs()
            for nd in [loss] + keep[::-1]:
                nd.release()
            return out
        finally:
            tlib.tth_conv_chain(prev)

    print("chain softmax-CE recipe, read", when, flush=True)
    got = run(True, when)
    if when == "never":
        got = run(True, "after")  # the next step after a graph released unread
    want = run(False, "after")
    for k in got:
        assert np.abs(got[k] - want[k]).max() <= 1e-4 * max(1e-30, np.abs(want[k]).max()), k
    assert abs(float(got["loss"][0]) - ref["loss"]) <= 1e-4 * max(1.0, abs(ref["loss"]))
    assert np.abs(got["probs"] - ref["probs"]).max() <= 1e-4


def test_autograd_chain_ce_in_head_bitexact(tlib):
    """The softmax-CE the classifier backward forms itself (two lanes a row,
    ce_row_pair) gives the bits the reduction kernel (ce_row, one lane a row)
    gives: the loss, probabilities and every gradient with the recipe read
    before the backward (the reduction runs) and after it (the head forms
    them) are equal bit for bit."""
    from tinytorch_amd.torch_py import Node
    x, y, P = orc.cnn_inputs(B=128)
    y = y.copy()
    y[::17] = 12  # labels outside [0, 10): the loss of ce_row's rule

    def run(read_first):
        keep = []
        logits = _cnn(Node, x, P, keep)
        loss = logits.softmax_ce(y)
        out = {}
        if read_first:
            out["probs"] = loss.probs()
        loss.backward(None)
        out["loss"] = loss.value()
        out["probs2"] = loss.probs()
        out["logits"] = logits.value()
        for k, i in (("dwfc", 5), ("dw2", 3), ("db2", 4), ("dw1", 1), ("db1", 2)):
            out[k] = keep[i].grad()
        for nd in [loss] + keep[::-1]:
            nd.release()
        return out

    print("chain CE in head vs reduction", flush=True)
    a, b = run(True), run(False)
    for k in b:
        assert bits_equal(a[k], b[k]), k
    assert bits_equal(a["probs"], b["probs2"])


@pytest.mark.parametrize("deferral", [True, False])
def test_classifier_backward_input_gradients_recipes(tlib, deferral):
    """The classifier backward with the second pool's backward in its launch
    leaves the reshape's and the pool's own gradients (dA without its ones
    column) as recipes of dA: read after the backward (and after the
    convolution's gradient was consumed), each equals dA[:, :-1] bit for bit;
    with every deferral off (tth_conv_relu_fuse(0)) the same gradients come
    from the unfused rules, within the fp32 bar of the fused ones."""
    from tinytorch_amd.torch_py import Node
    x, y, P = orc.cnn_inputs(B=128)

    def run(defer):
        prev = tlib.tth_conv_relu_fuse(1 if defer else 0)
        keep = []
        try:
            logits = _cnn(Node, x, P, keep)
            loss = logits.softmax_ce(y)
            loss.backward(None)
            names = ("X", "w1", "b1", "w2", "b2", "wfc", "c1", "r1", "p1", "c2", "r2", "p2", "f",
                     "d", "logits")
            g = {k: keep[names.index(k)].grad() for k in ("w2", "d", "f", "p2", "c2")}
            for nd in [loss] + keep[::-1]:
                nd.release()
            return g
        finally:
            tlib.tth_conv_relu_fuse(prev)

    print("classifier backward input gradient recipes, deferral", deferral, flush=True)
    g = run(deferral)
    dA = g["d"]
    assert bits_equal(g["f"], dA[:, :-1])
    assert bits_equal(g["p2"].reshape(128, -1), dA[:, :-1])
    if not deferral:
        return
    ref = run(False)
    for k in ("d", "f", "p2", "c2", "w2"):
        assert np.abs(g[k] - ref[k]).max() <= 1e-4 * max(1e-30, np.abs(ref[k]).max()), k
