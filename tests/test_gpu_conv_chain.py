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
    snap = DevBuf(32 * K1 + 32 + 18432 + 64)
    check(tlib.tt_k_conv2d_chain_fwd(dx.ptr, dw1.ptr, bp1, dw2.ptr, bp2, s1.ptr, j1.ptr, s2.ptr,
                                     e2.ptr, f2.ptr, j2.ptr, snap.ptr, N, C1, 32, 32, 32, 64),
          "chain")
    assert bits_equal(p1.to_np((N, 32, 16, 16)), s1.to_np((N, 32, 16, 16)))
    assert bits_equal(p2.to_np((N, 64, 8, 8)), s2.to_np((N, 64, 8, 8)))
    assert bits_equal(e2.to_np((N, 4096)), flat)
    assert bits_equal(f2.to_np((N, 4097)), orc.padones_fwd(flat))
    assert bits_equal(j1.to_np((N, 32, 16, 16)), k1)
    assert bits_equal(j2.to_np((N, 64, 8, 8)), k2)
    sn = snap.to_np((snap.n,))
    zb1 = b1 if bias else np.zeros(32, np.float32)
    zb2 = b2 if bias else np.zeros(64, np.float32)
    assert bits_equal(sn, np.concatenate([w1.ravel(), zb1, w2.ravel(), zb2]))
    # optional outputs left out: the rest unchanged
    s1b, j1b, s2b, j2b = DevBuf(p1n), DevBuf(p1n, np.uint8), DevBuf(p2n), DevBuf(p2n, np.uint8)
    check(tlib.tt_k_conv2d_chain_fwd(dx.ptr, dw1.ptr, bp1, dw2.ptr, bp2, s1b.ptr, j1b.ptr, s2b.ptr,
                                     None, None, j2b.ptr, None, N, C1, 32, 32, 32, 64),
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
                                      None, d.ptr, None, 2, 5, 32, 32, 32, 64) == -1
    assert tlib.tt_k_conv2d_chain_fwd(d.ptr, d.ptr, None, d.ptr, None, d.ptr, d.ptr, d.ptr, None,
                                      None, d.ptr, None, 2, 3, 16, 16, 32, 64) == -1
