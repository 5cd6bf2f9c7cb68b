"""A matmul and the layer after it in one GEMM + reduction pass.

tt_k_gemm_relu_pad must give exactly what tt_k_gemm followed by
tt_k_relu_padones_fwd gives (C, relu(C) and [relu(C), 1]), and those values
must be the oracle's relu / padones of C.  Shapes cover the split-K path
(the reduction carries the epilogue) and the paths without a reduction (the
epilogue runs as its own pass).  Also the softmax-CE with one-byte labels in
the launch arguments against the oracle.
"""
import ctypes

import numpy as np
import pytest

import orc
from tinytorch_amd.hip import DevBuf, check

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(4242)


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


RELU_SHAPES = [(256, 785, 512), (256, 513, 256), (64, 3000, 100), (7, 9, 5), (1, 1, 1),
               (300, 4096, 1000)]


@pytest.mark.parametrize("M,K,N", RELU_SHAPES)
def test_gemm_relu_pad_matches_unfused(tlib, M, K, N):
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    dA, dB = DevBuf.from_np(A), DevBuf.from_np(B)
    C1, R1, P1 = DevBuf(M * N), DevBuf(M * N), DevBuf(M * (N + 1))
    C2, R2, P2 = DevBuf(M * N), DevBuf(M * N), DevBuf(M * (N + 1))
    print("gemm_relu_pad", M, K, N, flush=True)
    check(tlib.tt_k_gemm_relu_pad(M, N, K, dA.ptr, dB.ptr, C1.ptr, R1.ptr, P1.ptr), "fused")
    check(tlib.tt_k_gemm(M, N, K, dA.ptr, K, 0, dB.ptr, N, 0, C2.ptr, N), "gemm")
    check(tlib.tt_k_relu_padones_fwd(C2.ptr, R2.ptr, P2.ptr, M, N), "relu_padones")
    c = C1.to_np((M, N))
    assert bits_equal(c, C2.to_np((M, N)))
    assert bits_equal(R1.to_np((M, N)), R2.to_np((M, N)))
    assert bits_equal(P1.to_np((M, N + 1)), P2.to_np((M, N + 1)))
    # and what the values are: relu and a column of ones
    assert bits_equal(R1.to_np((M, N)), orc.relu_fwd(c))
    assert bits_equal(P1.to_np((M, N + 1)), orc.padones_fwd(orc.relu_fwd(c)))


def test_gemm_relu_pad_rejects(tlib):
    d = DevBuf(64)
    assert tlib.tt_k_gemm_relu_pad(0, 1, 1, d.ptr, d.ptr, d.ptr, d.ptr, d.ptr) == -1
    assert tlib.tt_k_gemm_relu_pad(1, 1, 1, d.ptr, d.ptr, d.ptr, None, d.ptr) == -1


CE_CASES = [(128, 10), (256, 10), (33, 17), (512, 32), (5, 3), (300, 300)]


@pytest.mark.parametrize("rows,cols", CE_CASES)
def test_softmax_ce_hostlab_u8_labels(tlib, rows, cols):
    """Labels travel inside the launch arguments, one byte each for up to 255
    columns: labels outside [0, cols) (-1, cols, 300) must still give the
    loss -log(1e-12) and no one-hot term, as with 4-byte labels."""
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 3
    y = rng.integers(0, cols, rows).astype(np.int32)
    if rows >= 4:
        y[:4] = [-1, cols, 300, cols - 1]
    yp = y.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    dx, p, s, l = DevBuf.from_np(x), DevBuf(rows * cols), DevBuf(rows * cols), DevBuf(1)
    print("ce hostlab", rows, cols, flush=True)
    check(tlib.tt_k_softmax_ce_mean_hostlab(dx.ptr, yp, p.ptr, l.ptr, s.ptr, rows, cols,
                                            ctypes.c_float(1.0 / rows)), "ce")
    probs = orc.softmax_fwd(x)
    loss, seed = orc.ce_seed(probs, y)
    assert np.abs(p.to_np((rows, cols)) - probs).max() <= 1e-6
    assert abs(float(l.to_np((1,))[0]) - loss) <= 1e-5 * max(1.0, abs(loss))
    assert np.abs(s.to_np((rows, cols)) - seed).max() <= 1e-6


PAIR_SHAPES = [(256, 513, 256), (128, 1025, 160), (384, 417, 352)]


@pytest.mark.parametrize("M,K,N", PAIR_SHAPES)
@pytest.mark.parametrize("mode", ["plain", "copy", "relu"])
def test_matmul_bwd_small_matches_two_gemms(tlib, M, K, N, mode):
    """Both gradients in one launch: dA and dB bit-identical to the two
    tt_k_gemm calls of the unfused rule, d1 / d2 the padones (relu) backward
    of dA exactly; within tolerance of the oracle's matmul_nt / matmul_tn."""
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    G = (rng.standard_normal((M, N)) / M).astype(np.float32)
    R = np.maximum(rng.standard_normal((M, K - 1)).astype(np.float32), 0.0)
    dA_, dB_, dG, dR = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf.from_np(G), DevBuf.from_np(R)
    gb, ga, d1, d2 = DevBuf(K * N), DevBuf(M * K), DevBuf(M * (K - 1)), DevBuf(M * (K - 1))
    rb, ra = DevBuf(K * N), DevBuf(M * K)
    print("matmul_bwd_small", M, K, N, mode, flush=True)
    rc = tlib.tt_k_matmul_bwd_small(dA_.ptr, M, K, dB_.ptr, N, dG.ptr, gb.ptr, ga.ptr,
                                    d1.ptr if mode != "plain" else None,
                                    d2.ptr if mode != "plain" else None,
                                    dR.ptr if mode == "relu" else None)
    if rc == -1:
        pytest.skip("tt_k_gemm takes another kernel for this shape")
    check(rc, "tt_k_matmul_bwd_small")
    check(tlib.tt_k_gemm(M, K, N, dG.ptr, N, 0, dB_.ptr, N, 1, ra.ptr, K), "dA")
    check(tlib.tt_k_gemm(K, N, M, dA_.ptr, K, 1, dG.ptr, N, 0, rb.ptr, N), "dB")
    a, b = ga.to_np((M, K)), gb.to_np((K, N))
    assert bits_equal(a, ra.to_np((M, K)))
    assert bits_equal(b, rb.to_np((K, N)))
    if mode != "plain":
        assert bits_equal(d1.to_np((M, K - 1)), a[:, :-1])
        want2 = orc.relu_bwd(R, a[:, :-1]) if mode == "relu" else a[:, :-1]
        assert bits_equal(d2.to_np((M, K - 1)), want2)
    ea = orc.matmul_nt(G, B)
    eb = orc.matmul_tn(A, G)
    assert np.abs(a - ea).max() <= 1e-5 * max(1.0, np.abs(ea).max())
    assert np.abs(b - eb).max() <= 1e-5 * max(1.0, np.abs(eb).max())


def test_matmul_bwd_small_shapes_taken(tlib):
    """The MLP's middle layer (config 2: 256 x 513 x 256) is covered."""
    d = DevBuf(256 * 513)
    g = DevBuf(256 * 256)
    w = DevBuf(513 * 256)
    assert tlib.tt_k_matmul_bwd_small(d.ptr, 256, 513, w.ptr, 256, g.ptr, DevBuf(513 * 256).ptr,
                                      DevBuf(256 * 513).ptr, None, None, None) == 0


# (the first two and (250, 780, 500) .. (1000, 64, 250) take the 16x16-tile
# kernel: ragged M and N, K not a multiple of a wave's slice, waves with no
# k at all; (128, 4096, 10) and the last three its split-K form for skinny
# outputs: ragged rows, K not a multiple of a slice, 1 to 63 row tiles;
# (100, 30, 7) the 16-row classifier tiles with unaligned rows; (256, 784,
# 512) and (250, 500, 1000) the 16x32 tiles, the latter with a ragged last
# column block)
BIAS_SHAPES = [(256, 784, 512), (256, 512, 256), (256, 256, 10), (128, 4096, 10), (7, 9, 5),
               (300, 1000, 96), (64, 3, 40), (250, 780, 500), (256, 20, 300), (1000, 64, 250),
               (100, 2048, 7), (1000, 3000, 3), (16, 4100, 16), (100, 30, 7), (250, 500, 1000),
               # the skinny split-K kernel's other chunk counts per wave:
               # 16, 8, 2, 3, 4, 5 (run as 6) and 7 (run as 8) chunks of 16 k
               (2048, 4096, 10), (1024, 4096, 16), (512, 2048, 16), (512, 3072, 10),
               (512, 4096, 10), (1024, 2560, 10), (1024, 3584, 12)]


@pytest.mark.parametrize("M,K,N", BIAS_SHAPES)
@pytest.mark.parametrize("epi", [False, True])
def test_gemm_bias_relu_pad_vs_padded_product(tlib, M, K, N, epi):
    """tt_k_gemm_bias_relu_pad (X * W[:K] + W[K], the matmul of a padones
    output from the padones input): C within the GEMM bar of the oracle's
    product of the padded matrix, and R / P exactly relu(C) / [relu(C), 1]."""
    X = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    W = (rng.standard_normal((K + 1, N)) / np.sqrt(K)).astype(np.float32)
    dX, dW = DevBuf.from_np(X), DevBuf.from_np(W)
    bias_ptr = dW.ptr + 4 * K * N
    C, R, P = DevBuf(M * N), DevBuf(M * N), DevBuf(M * (N + 1))
    print("gemm_bias_relu_pad", M, K, N, epi, flush=True)
    check(tlib.tt_k_gemm_bias_relu_pad(M, N, K, dX.ptr, dW.ptr, bias_ptr, C.ptr,
                                       R.ptr if epi else None, P.ptr if epi else None), "bias")
    c = C.to_np((M, N))
    ref = orc.sgemm(orc.padones_fwd(X), W)
    amax = max(1.0, float(np.abs(W).max()))
    assert np.abs(c - ref).max() / (np.sqrt(K + 1) * amax) <= 1e-4
    if epi:
        assert bits_equal(R.to_np((M, N)), orc.relu_fwd(c))
        assert bits_equal(P.to_np((M, N + 1)), orc.padones_fwd(orc.relu_fwd(c)))


@pytest.mark.parametrize("M,K,N", [(256, 784, 512), (128, 4096, 10), (256, 256, 10),
                                   (2048, 4096, 10), (1024, 4096, 16), (512, 2048, 16)])
def test_gemm_bias_t16_off_same_bar(tlib, M, K, N):
    """With the 16x16-tile kernels switched off (tth_gemm_t16(0)) the same
    shapes take the split-K / row kernels: C within the GEMM bar of the
    oracle either way."""
    X = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    W = (rng.standard_normal((K + 1, N)) / np.sqrt(K)).astype(np.float32)
    dX, dW = DevBuf.from_np(X), DevBuf.from_np(W)
    bias_ptr = dW.ptr + 4 * K * N
    ref = orc.sgemm(orc.padones_fwd(X), W)
    amax = max(1.0, float(np.abs(W).max()))
    out = []
    print("gemm_bias t16 on/off", M, K, N, flush=True)
    try:
        for on in (1, 0):
            check(tlib.tth_gemm_t16(on), "t16")
            C = DevBuf(M * N)
            check(tlib.tt_k_gemm_bias_relu_pad(M, N, K, dX.ptr, dW.ptr, bias_ptr, C.ptr, None,
                                               None), "bias")
            out.append(C.to_np((M, N)))
    finally:
        check(tlib.tth_gemm_t16(1), "t16 on")
    for c in out:
        assert np.abs(c - ref).max() / (np.sqrt(K + 1) * amax) <= 1e-4


# (rows, Kx, N, taken): the MLP's first layer (784 -> 512 at batch 256),
# ragged widths, and a shape the small-GEMM tiles do not take (too few
# tiles: -1, nothing launched)
TN_PAD_SHAPES = [(256, 784, 512, True), (200, 1023, 300, True), (512, 390, 700, True),
                 (300, 33, 257, False)]


@pytest.mark.parametrize("rows,Kx,N,taken", TN_PAD_SHAPES)
def test_gemm_tn_padones_bitexact(tlib, rows, Kx, N, taken):
    """[X, 1]^T G from X: bit for bit tt_k_gemm on the padded matrix (the
    ones row is the column sums of G), and within tolerance of float64."""
    x = np.random.default_rng(5).uniform(-1, 1, (rows, Kx)).astype(np.float32)
    g = np.random.default_rng(6).standard_normal((rows, N)).astype(np.float32)
    xp = orc.padones_fwd(x)
    dx_, dxp, dg = DevBuf.from_np(x), DevBuf.from_np(xp), DevBuf.from_np(g)
    d1, d2 = DevBuf((Kx + 1) * N), DevBuf((Kx + 1) * N)
    print("gemm_tn_padones", rows, Kx, N, flush=True)
    rc = tlib.tt_k_gemm_tn_padones(rows, Kx, N, dx_.ptr, dg.ptr, d1.ptr)
    if not taken:
        assert rc == -1
        return
    check(rc, "gemm_tn_padones")
    check(tlib.tt_k_gemm(Kx + 1, N, rows, dxp.ptr, Kx + 1, 1, dg.ptr, N, 0, d2.ptr, N), "gemm")
    got = d1.to_np((Kx + 1, N))
    assert np.array_equal(got.view(np.uint32), d2.to_np((Kx + 1, N)).view(np.uint32))
    ref = xp.astype(np.float64).T @ g.astype(np.float64)
    assert np.abs(got - ref).max() / np.sqrt(rows) <= 1e-4 * np.abs(g).max()


def test_gemm_tn_padones_rejects(tlib):
    d = DevBuf(16)
    assert tlib.tt_k_gemm_tn_padones(0, 4, 4, d.ptr, d.ptr, d.ptr) == -1
    # 4096-row output: the big tiles, not the small-GEMM kernel (buffers of
    # the full sizes all the same)
    x, g, dw = DevBuf(4096 * 4095), DevBuf(4096 * 4096), DevBuf(4096 * 4096)
    assert tlib.tt_k_gemm_tn_padones(4096, 4095, 4096, x.ptr, g.ptr, dw.ptr) == -1


@pytest.mark.parametrize("read_first", [False, True])
def test_autograd_padones_input_unpadded(tlib, read_first):
    """padones of an input that needs no gradient feeding a matmul (the
    MLP's first layer): the padded copy is written only when read, the
    weight gradient comes from the input itself -- values and gradients bit
    for bit those of the graph with every launch made at once."""
    from tinytorch_amd.torch_py import Node
    rng = np.random.default_rng(8)
    x = rng.uniform(0, 1, (256, 784)).astype(np.float32)
    w = (rng.standard_normal((785, 512)) * 0.05).astype(np.float32)
    gy = rng.standard_normal((256, 512)).astype(np.float32)

    def run():
        X, Wn = Node.leaf(x, False), Node.leaf(w)
        P = X.padones()
        pv = P.value() if read_first else None
        Y = P.matmul(Wn)
        yv = Y.value()
        Y.backward(gy)
        out = [yv, Wn.grad(), P.value()]
        if read_first:
            assert np.array_equal(pv, out[2])
        for nd in (Y, P, X, Wn):
            nd.release()
        return out

    prev = tlib.tth_conv_relu_fuse(0)
    try:
        ref = run()
    finally:
        tlib.tth_conv_relu_fuse(prev)
    got = run()
    for a, e in zip(got, ref):
        assert np.array_equal(a.view(np.uint32), e.view(np.uint32))
    assert np.array_equal(got[2], orc.padones_fwd(x))


# (M, N, K): the CNN classifier (128 x 4096 -> 10), the MLP's last layer
# (256 x 256 -> 10), wider rows, and a shape whose GEMM takes no split-K path
CE_SHAPES = [(128, 10, 4096), (256, 10, 256), (100, 32, 2000), (7, 3, 4100), (512, 10, 64),
             (33, 10, 8192), (200, 16, 2052), (2048, 10, 4096), (1024, 16, 4096), (512, 16, 2048)]


@pytest.mark.parametrize("M,N,K", CE_SHAPES)
def test_gemm_bias_ce_matches_unfused(tlib, M, N, K):
    """The softmax-CE inside the classifier GEMM's split-K reduction: logits,
    probabilities, seed and (through tt_k_ce_mean_rows) the mean loss bit for
    bit those of the GEMM followed by the one-workgroup softmax-CE kernel;
    labels out of range included.  Return 1 (a GEMM without split-K): the
    logits only."""
    r = np.random.default_rng(11)
    a = r.uniform(-1, 1, (M, K)).astype(np.float32)
    b = (r.standard_normal((K, N)) * 0.1).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    y = r.integers(0, N, M).astype(np.int32)
    y[::13] = N + 2
    da, db, dbias = DevBuf.from_np(a), DevBuf.from_np(b), DevBuf.from_np(bias)
    c1, p1, s1, rl, l1 = DevBuf(M * N), DevBuf(M * N), DevBuf(M * N), DevBuf(M), DevBuf(1)
    c2, p2, s2, l2 = DevBuf(M * N), DevBuf(M * N), DevBuf(M * N), DevBuf(1)
    scale = ctypes.c_float(1.0 / M)
    print("gemm_bias_ce", M, N, K, flush=True)
    rc = tlib.tt_k_gemm_bias_ce(M, N, K, da.ptr, db.ptr, dbias.ptr, c1.ptr, y.ctypes.data,
                                p1.ptr, s1.ptr, rl.ptr, scale)
    assert rc in (0, 1), rc
    check(tlib.tt_k_gemm_bias_relu_pad(M, N, K, da.ptr, db.ptr, dbias.ptr, c2.ptr, None, None),
          "gemm bias")
    assert bits_equal(c1.to_np((M, N)), c2.to_np((M, N)))
    if (M, N, K) in ((128, 10, 4096), (256, 10, 256)):
        assert rc == 0  # the two configs' classifiers take split-K
    if rc == 1:
        return
    check(tlib.tt_k_softmax_ce_mean_hostlab(c2.ptr, y.ctypes.data, p2.ptr, l2.ptr, s2.ptr, M, N,
                                            scale), "ce")
    check(tlib.tt_k_ce_mean_rows(rl.ptr, l1.ptr, M), "mean")
    assert bits_equal(p1.to_np((M, N)), p2.to_np((M, N)))
    assert bits_equal(s1.to_np((M, N)), s2.to_np((M, N)))
    assert bits_equal(l1.to_np((1,)), l2.to_np((1,)))


@pytest.mark.parametrize("read_loss", ["before", "after", "never"])
def test_autograd_classifier_ce_in_reduction(tlib, read_loss):
    """padones -> matmul -> softmax_ce (the classifier layer): the CE joins
    the pending GEMM's reduction and the mean loss is written when read --
    loss, logits, probabilities and gradients bit for bit those of the same
    graph whose logits are read before the softmax-CE (the GEMM then runs by
    itself and the one-workgroup CE kernel after it)."""
    from tinytorch_amd.torch_py import Node
    r = np.random.default_rng(12)
    x = r.uniform(0, 1, (128, 4096)).astype(np.float32)
    w = (r.standard_normal((4097, 10)) * 0.02).astype(np.float32)
    y = r.integers(0, 10, 128)

    def run(join):
        X, Wn = Node.leaf(x), Node.leaf(w)
        P = X.padones()
        Z = P.matmul(Wn)
        if not join:
            Z.value()
        L = Z.softmax_ce(y)
        out = []
        if read_loss == "before":
            out.append(L.value())
        L.backward(None)
        if read_loss == "after":
            out.append(L.value())
        out += [Z.value(), Wn.grad(), X.grad()]
        for nd in (L, Z, P, X, Wn):
            nd.release()
        return out

    ref = run(False)
    got = run(True)
    for g, e in zip(got, ref):
        assert bits_equal(g, e)
    wp = np.concatenate([x, np.ones((128, 1), np.float32)], 1)
    z = wp.astype(np.float64) @ w.astype(np.float64)
    p = np.exp(z - z.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    if read_loss != "never":
        loss = -np.log(p[np.arange(128), y]).mean()
        assert abs(float(got[0][0]) - loss) <= 1e-4 * max(1.0, abs(loss))


def test_recipe_source_written_through_host_pointer(tlib):
    """A tensor left as a recipe (the padded copy of a no-grad input) is
    written before the host may change its source: tt_data of the source
    runs the recipe first, so the padded copy keeps the values the input had
    when ag_padones was called."""
    from tinytorch_amd.torch_py import Node
    x = np.random.default_rng(21).uniform(-1, 1, (64, 96)).astype(np.float32)
    X = Node.leaf(x, False)
    P = X.padones()
    xt = tlib.ag_value(X.ptr)
    hp = tlib.tt_data(xt)
    assert hp
    buf = np.ctypeslib.as_array(ctypes.cast(hp, ctypes.POINTER(ctypes.c_float)), shape=(x.size,))
    buf[:] = 5.0  # the caller writes the input through the host pointer
    assert np.array_equal(P.value(), orc.padones_fwd(x))
    assert np.all(X.value() == 5.0)
    for nd in (P, X):
        nd.release()


@pytest.mark.parametrize("second_pass", [False, True])
def test_mlp_first_layer_grad_pending_into_sgd(tlib, second_pass):
    """The first layer's weight gradient of padones(X) -> matmul (X without
    gradient) is left pending and computed inside the SGD step's launch (the
    step of its weights in the same threads): the stepped weights and the
    gradients bit for bit those of reading the gradients first; a second
    backward pass before the step (which adds into the layer's output
    gradient the recipe reads) gives the same bits both ways too."""
    from tinytorch_amd.torch_py import Node
    r = np.random.default_rng(51)
    x = r.uniform(0, 1, (256, 784)).astype(np.float32)
    w1 = (r.standard_normal((785, 512)) * 0.05).astype(np.float32)
    w2 = (r.standard_normal((513, 10)) * 0.05).astype(np.float32)
    gy = r.standard_normal((256, 10)).astype(np.float32)

    def run(read_first):
        X, W1, W2 = Node.leaf(x, False), Node.leaf(w1), Node.leaf(w2)
        P1 = X.padones()
        H = P1.matmul(W1).relu()
        P2 = H.padones()
        Y = P2.matmul(W2)
        Y.backward(gy)
        if second_pass:
            Y.backward(gy)
        if read_first:
            W1.grad()
        arr = (ctypes.c_void_p * 2)(W1.ptr, W2.ptr)
        assert tlib.ag_sgd_step_many(arr, 2, ctypes.c_float(0.05)) == 0
        out = [W1.value(), W2.value(), W1.grad(), W2.grad()]
        for nd in (Y, P2, H, P1, X, W1, W2):
            nd.release()
        return out

    fused, plain = run(False), run(True)
    for a, b in zip(fused, plain):
        assert bits_equal(a, b)
    if second_pass:
        return  # (a second pass re-propagates the accumulated intermediate gradients)
    # the gradient itself against float64
    xp = orc.padones_fwd(x).astype(np.float64)
    h = np.maximum(xp @ w1, 0.0)
    gh = (gy.astype(np.float64) @ w2[:512].astype(np.float64).T) * (h > 0)
    want = xp.T @ gh
    e = np.abs(fused[2] - want).max() / np.abs(want).max()
    assert e <= 1e-4, e


@pytest.mark.parametrize("read_first", [False, True])
def test_sgd_step_of_a_tensor_a_pending_gradient_reads(tlib, read_first):
    """One tensor T is both a trained leaf and, through a no-gradient leaf
    sharing it (`detach`), the padones input of a matmul whose weight
    gradient [T, 1]^T G stays pending.  The SGD step that updates T must run
    that gradient from T's values before the update: the stepped weights
    equal w - lr * [T, 1]^T G within the GEMM bar of float64, and bit for bit
    the weights of reading every gradient before the step."""
    from tinytorch_amd.torch_py import Node
    r = np.random.default_rng(61)
    M, K, N = 256, 784, 512
    t = r.uniform(0, 1, (M, K)).astype(np.float32)
    w = (r.standard_normal((K + 1, N)) * 0.05).astype(np.float32)
    v = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
    g = r.standard_normal((M, N)).astype(np.float32)
    lr = 0.5

    def run(read):
        T = Node.leaf(t)
        X = T.detach(False)
        Wn, Vn = Node.leaf(w), Node.leaf(v, False)
        P = X.padones()
        A, B = P.matmul(Wn), T.matmul(Vn)
        Y = A + B
        Y.backward(g)
        if read:
            Wn.grad(), T.grad()
        arr = (ctypes.c_void_p * 2)(Wn.ptr, T.ptr)
        assert tlib.ag_sgd_step_many(arr, 2, ctypes.c_float(lr)) == 0
        out = [Wn.value(), T.value()]
        for nd in (Y, A, B, P, X, Wn, Vn, T):
            nd.release()
        return out

    print("sgd step of a tensor a pending gradient reads, read_first", read_first, flush=True)
    got = run(read_first)
    if not read_first:
        for a, e in zip(got, run(True)):
            assert bits_equal(a, e)
    tp = orc.padones_fwd(t).astype(np.float64)
    dw = tp.T @ g.astype(np.float64)
    dt = g.astype(np.float64) @ v.astype(np.float64).T
    bar_w = lr * 1e-4 * np.sqrt(M) * np.abs(g).max() + np.spacing(np.abs(w).max())
    bar_t = lr * 1e-4 * np.sqrt(N) * np.abs(g).max() * np.abs(v).max() + np.spacing(1.0)
    assert np.abs(got[0] - (w - lr * dw)).max() <= bar_w
    assert np.abs(got[1] - (t - lr * dt)).max() <= bar_t


@pytest.mark.parametrize("case", ["default", "seed2", "twice", "frozen_w2", "w2_written"])
def test_classifier_input_grads_formed_with_the_seed(tlib, case):
    """relu -> padones -> matmul -> softmax_ce (the MLP's last layer): the
    classifier's launch also forms, from each row's seed, the gradients of
    the padones node, the relu and its input (the classifier backward's dA,
    bit for bit); the backward takes them when it starts from this loss with
    the default seed, the weights' gradient then being a recipe of the
    optimizer's launch.  Every node gradient is compared with the same graph
    whose logits are read before the softmax-CE (no such launch: the
    classifier backward kernel): bit for bit, except the classifier weights'
    gradient (MFMA tiles against the backward kernel's serial sums: within
    1e-5 of its scale).  A seed of 2, a second backward (accumulating) and
    frozen classifier weights, or weights written between the passes, leave
    the backward its own kernel."""
    from tinytorch_amd.torch_py import Node
    r = np.random.default_rng(21)
    x = r.uniform(0, 1, (256, 100)).astype(np.float32)
    w1 = (r.standard_normal((101, 64)) * 0.1).astype(np.float32)
    w2 = (r.standard_normal((65, 10)) * 0.2).astype(np.float32)
    y = r.integers(0, 10, 256)

    def run(read_logits, seed=None, twice=False, w2_grad=True, write_w2=False):
        X, W1, W2 = Node.leaf(x, False), Node.leaf(w1), Node.leaf(w2, w2_grad)
        P1 = X.padones()
        H = P1.matmul(W1)
        R = H.relu()
        P2 = R.padones()
        Z = P2.matmul(W2)
        if read_logits:
            Z.value()
        L = Z.softmax_ce(y)
        if write_w2:
            # the classifier weights changed through their host copy between
            # the forward and the backward pass
            t = tlib.ag_value(W2.ptr)
            hp = tlib.tt_data(t)
            np.ctypeslib.as_array(hp, shape=(w2.size,))[:] *= np.float32(0.5)
        L.backward(seed)
        if twice:
            L.backward(seed)
        out = dict(loss=L.value(), z=Z.value(), w1=W1.grad(), h=H.grad(), r=R.grad(),
                   p2=P2.grad(), w2=W2.grad())
        for nd in (L, Z, P2, R, H, P1, X, W1, W2):
            nd.release()
        return out

    print("classifier input grads with the seed:", case, flush=True)
    kw = dict(default={}, seed2=dict(seed=np.array([2.0], np.float32)), twice=dict(twice=True),
              frozen_w2=dict(w2_grad=False), w2_written=dict(write_w2=True))[case]
    n0 = tlib.tth_ce_spec_count()
    got = run(False, **kw)
    taken = tlib.tth_ce_spec_count() - n0
    assert taken == (1 if case in ("default", "twice") else 0), taken
    ref = run(True, **kw)
    assert tlib.tth_ce_spec_count() - n0 == taken
    assert bits_equal(got["loss"], ref["loss"]) and bits_equal(got["z"], ref["z"])
    for name in ("w1", "h", "r", "p2"):
        assert bits_equal(got[name], ref[name]), name
    if case == "frozen_w2":
        assert got["w2"] is None
    elif case in ("seed2", "w2_written"):
        # not taken: the same kernel on both sides
        assert bits_equal(got["w2"], ref["w2"])
    else:
        assert np.abs(got["w2"] - ref["w2"]).max() <= 1e-5 * np.abs(ref["w2"]).max()


def test_classifier_and_first_layer_grads_in_one_sgd_launch(tlib):
    """The MLP's two pending padones weight gradients (first layer and
    classifier) and the plain step of the middle layer in one optimizer
    launch: every weight equals w - lr * g, g the gradient of the same graph
    read before stepping (each pending gradient formed by its own launch)."""
    from tinytorch_amd.torch_py import Node
    r = np.random.default_rng(22)
    x = r.uniform(0, 1, (256, 784)).astype(np.float32)
    ws = [(r.standard_normal(s) * 0.05).astype(np.float32) for s in ((785, 128), (129, 64), (65, 10))]
    y = r.integers(0, 10, 256)
    lr = 0.05

    def run(read_grads):
        X = Node.leaf(x, False)
        W = [Node.leaf(w) for w in ws]
        h = X.padones().matmul(W[0]).relu().padones().matmul(W[1]).relu().padones()
        L = h.matmul(W[2]).softmax_ce(y)
        L.backward(None)
        g = [w.grad() for w in W] if read_grads else None
        arr = (ctypes.c_void_p * 3)(*[w.ptr for w in W])
        check(tlib.ag_sgd_step_many(arr, 3, ctypes.c_float(lr)), "sgd many")
        out = [w.value() for w in W], g
        L.release()
        X.release()
        for w in W:
            w.release()
        return out

    print("sgd launch with two pending padones gradients", flush=True)
    stepped, _ = run(False)
    ref_w, g = run(True)
    for i in range(3):
        assert bits_equal(ref_w[i], ws[i] - np.float32(lr) * g[i]), i
        assert bits_equal(stepped[i], ref_w[i]), i



def test_classifier_input_grads_taken_in_the_mlp_step(tlib):
    """The bench's config-2 step (and the test graph above) take the
    classifier's input gradients formed with the seed: the library's count of
    such backward rules goes up by one a step."""
    import bench
    st = bench.MlpStep(tlib)
    n0 = tlib.tth_ce_spec_count()
    st.step()
    st.step(lr=0.01)
    assert tlib.tth_ce_spec_count() == n0 + 2
