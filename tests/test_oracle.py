"""Pins the CPU oracle (oracle/orc.c) before it is trusted as the GPU checker.

Three independent pins, so that a dropped term, a wrong index or a
transposed operand in the restatement fails at least one:
  1. bit-for-bit against the reference library compiled from its own
     sources (oracle/_ref), when that build exists;
  2. bit-for-bit against the committed golden vectors written from that
     build (tests/golden/ref_vectors.npz), always;
  3. against mathematics: float64 products, brute-force index maps, the
     im2col/col2im adjoint identity, closed-form special cases and central
     finite differences of the backward rules.
"""
import os

import numpy as np
import pytest

import orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")
needs_ref = pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref not built")
rng = np.random.default_rng(1234)


def u(*s):
    return rng.uniform(-1, 1, s).astype(np.float32)


def same(a, b):
    """bitwise equality, NaN == NaN"""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------- 1. vs _ref

@needs_ref
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 3, 7), (6, 16, 20), (17, 13, 5), (64, 512, 16),
                                   (100, 70, 400), (130, 1040, 777), (9, 256, 33)])
def test_sgemm_bitexact_vs_ref(M, N, K):
    A, B = u(M, K), u(K, N)
    A[0, 0] = 0.0  # exercises the tails' a == 0 skip
    assert same(orc.sgemm(A, B), orc.ref_sgemm(A, B))


def naive_case(M=37, N=29, K=23):
    A, B = u(M, K), u(K, N)
    A[A < -0.6] = 0.0
    A[1, 2] = -0.0
    B[2, :5] = [np.nan, np.inf, -np.inf, np.nan, 1.0]   # row k=2 meets A[1,2] = -0.0
    A[3, 2] = 0.5                                       # ... and a non-zero: NaN/Inf reach row 3
    return A, B


@needs_ref
def test_matmul_naive_bitexact_vs_ref():
    """reference tt_matmul (src/ops.c:84-101) including its a == 0 skip"""
    A, B = naive_case()
    assert same(orc.matmul_naive(A, B), orc.ref_matmul(A, B))


def test_matmul_naive_zero_skip_and_float64():
    """A zero of A masks NaN / Inf in the matching row of B (the skip); a
    non-zero lets them through; finite entries equal the float64 product
    summed in k order with float32 rounding, which for small integers is
    exact."""
    A, B = naive_case()
    C = orc.matmul_naive(A, B)
    rows_hit = np.nonzero(A[:, 2] != 0)[0]
    assert 1 not in rows_hit and 3 in rows_hit
    assert np.isfinite(C[1]).all()
    assert np.isnan(C[3, 0]) and np.isnan(C[3, 3])
    assert C[3, 1] == np.inf and C[3, 2] == -np.inf
    # finite case: serial float32 accumulation
    Ai = rng.integers(-3, 4, (9, 11)).astype(np.float32)
    Bi = rng.integers(-3, 4, (11, 7)).astype(np.float32)
    assert same(orc.matmul_naive(Ai, Bi), (Ai.astype(np.float64) @ Bi).astype(np.float32))
    Af, Bf = u(8, 50), u(50, 6)
    ref = np.zeros((8, 6), np.float32)
    for k in range(50):
        nz = Af[:, k] != 0
        ref[nz] = ref[nz] + (Af[nz, k:k + 1] * Bf[k:k + 1, :])
    assert same(orc.matmul_naive(Af, Bf), ref)


@needs_ref
def test_matmul_grads_bitexact_vs_ref():
    A, B, G = u(33, 21), u(21, 19), u(33, 19)
    g = orc.RefGraph()
    L = orc.ref()
    nA, nB = g.leaf(A), g.leaf(B)
    g.backward(g.add(L.ag_matmul(nA, nB)), G)
    assert same(orc.matmul_nt(G, B), g.grad(nA, A.shape))
    assert same(orc.matmul_tn(A, G), g.grad(nB, B.shape))
    g.release()


@needs_ref
@pytest.mark.parametrize("sh,ph", [(1, 1), (1, 0), (2, 1), (2, 2)])
def test_conv_bitexact_vs_ref(sh, ph):
    x, w, b = u(3, 4, 9, 9), u(5, 4, 3, 3), u(5)
    y = orc.conv2d_fwd(x, w, b, sh, sh, ph, ph)
    G = u(*y.shape)
    g = orc.RefGraph()
    L = orc.ref()
    nx, nw, nb = g.leaf(x), g.leaf(w), g.leaf(b)
    ny = g.add(L.ag_conv2d(nx, nw, nb, sh, sh, ph, ph))
    assert same(y, g.value(ny, y.shape))
    g.backward(ny, G)
    dx, dw, db = orc.conv2d_bwd(x, w, G, sh, sh, ph, ph)
    assert same(dx, g.grad(nx, x.shape))
    assert same(dw, g.grad(nw, w.shape))
    assert same(db, g.grad(nb, b.shape))
    g.release()


@needs_ref
@pytest.mark.parametrize("p,s", [(2, 2), (3, 2), (2, 1), (3, 3)])
def test_pools_bitexact_vs_ref(p, s):
    x = u(2, 3, 8, 7)
    x[0, 0, :3, :3] = 0.25
    x[1, 1] = np.nan
    y = orc.maxpool_fwd(x, p, p, s, s)
    G = u(*y.shape)
    g = orc.RefGraph()
    L = orc.ref()
    nx = g.leaf(x)
    ny = g.add(L.ag_maxpool2d(nx, p, p, s, s))
    assert same(y, g.value(ny, y.shape))
    g.backward(ny, G)
    assert same(orc.maxpool_bwd(x, G, p, p, s, s), g.grad(nx, x.shape))
    g.release()
    xa = u(2, 3, 8, 7)
    g = orc.RefGraph()
    nx = g.leaf(xa)
    ny = g.add(L.ag_avgpool2d(nx, p, p, s, s))
    assert same(orc.avgpool_fwd(xa, p, p, s, s), g.value(ny, y.shape))
    g.backward(ny, G)
    assert same(orc.avgpool_bwd(G, xa.shape, p, p, s, s), g.grad(nx, xa.shape))
    g.release()


@needs_ref
def test_steps_bitexact_vs_ref():
    x, y, Ws = orc.mlp_inputs(B=32, dims=(50, 40, 30, 10), seed=5)
    o, r = orc.mlp_step(x, y, *Ws), orc.ref_mlp_step(x, y, *Ws)
    for k in ("logits", "probs", "dW1", "dW2", "dW3"):
        assert same(o[k], r[k]), k
    x, y, P = orc.cnn_inputs(B=8, H=16, W=16, F1=8, F2=16, seed=6)
    o, r = orc.cnn_step(x, y, **P), orc.ref_cnn_step(x, y, **P)
    for k in ("logits", "probs", "dw1", "db1", "dw2", "db2", "dwfc"):
        assert same(o[k], r[k]), k


# ---------------------------------------------------------------- 2. vs golden vectors

@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def test_golden_gemm(gold):
    for tag in ("g1", "g2", "g3"):
        assert same(orc.sgemm(gold[f"{tag}_A"], gold[f"{tag}_B"]), gold[f"{tag}_C"]), tag


def test_golden_matmul_grads(gold):
    assert same(orc.matmul_nt(gold["mm_G"], gold["mm_B"]), gold["mm_dA"])
    assert same(orc.matmul_tn(gold["mm_A"], gold["mm_G"]), gold["mm_dB"])


def test_golden_conv(gold):
    for tag, (s, p) in (("c1", (1, 1)), ("c2", (2, 0))):
        x, w, b, G = (gold[f"{tag}_{k}"] for k in "xwbG")
        assert same(orc.conv2d_fwd(x, w, b, s, s, p, p), gold[f"{tag}_y"])
        dx, dw, db = orc.conv2d_bwd(x, w, G, s, s, p, p)
        assert same(dx, gold[f"{tag}_dx"]) and same(dw, gold[f"{tag}_dw"])
        assert same(db, gold[f"{tag}_db"])


def test_golden_pools(gold):
    for tag, (p, s) in (("mp1", (2, 2)), ("mp2", (3, 2))):
        x, G = gold[f"{tag}_x"], gold[f"{tag}_G"]
        assert same(orc.maxpool_fwd(x, p, p, s, s), gold[f"{tag}_y"])
        assert same(orc.maxpool_bwd(x, G, p, p, s, s), gold[f"{tag}_dx"])
        xa = gold[f"a{tag}_x"]
        assert same(orc.avgpool_fwd(xa, p, p, s, s), gold[f"a{tag}_y"])
        assert same(orc.avgpool_bwd(G, xa.shape, p, p, s, s), gold[f"a{tag}_dx"])


def test_golden_rows(gold):
    assert same(orc.relu_fwd(gold["relu_x"]), gold["relu_y"])
    assert same(orc.relu_bwd(gold["relu_x"], gold["relu_G"]), gold["relu_dx"])
    assert same(orc.softmax_fwd(gold["sm_x"]), gold["sm_y"])
    assert same(orc.softmax_bwd(gold["sm_y"], gold["sm_G"]), gold["sm_dx"])
    assert same(orc.padones_fwd(gold["po_x"]), gold["po_y"])
    assert same(orc.padones_bwd(gold["po_G"]), gold["po_dx"])


def test_golden_steps(gold):
    o = orc.mlp_step(gold["mlp_x"], gold["mlp_y"], gold["mlp_W1"], gold["mlp_W2"], gold["mlp_W3"])
    for k in ("logits", "probs", "dW1", "dW2", "dW3"):
        assert same(o[k], gold[f"mlp_{k}"]), k
    P = {k: gold[f"cnn_{k}"] for k in ("w1", "b1", "w2", "b2", "wfc")}
    o = orc.cnn_step(gold["cnn_x"], gold["cnn_y"], **P)
    for k in ("logits", "probs", "dw1", "db1", "dw2", "db2", "dwfc"):
        assert same(o[k], gold[f"cnn_r_{k}"]), k


# ---------------------------------------------------------------- 3. vs mathematics

@pytest.mark.parametrize("M,N,K", [(7, 5, 3), (64, 48, 40), (200, 33, 513)])
def test_gemm_family_vs_float64(M, N, K):
    A, B = u(M, K), u(K, N)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    tol = 4 * np.sqrt(K) * np.finfo(np.float32).eps * max(1.0, np.abs(ref).max())
    assert np.abs(orc.sgemm(A, B) - ref).max() < tol
    G = u(M, N)
    assert np.abs(orc.matmul_nt(G, B) - G.astype(np.float64) @ B.T).max() < K * 1e-6 + tol
    assert np.abs(orc.matmul_tn(A, G) - A.T.astype(np.float64) @ G).max() < M * 1e-6 + tol
    Bt = np.ascontiguousarray(B.T)
    assert np.abs(orc.sgemm_a_bt(A, Bt) - ref).max() < tol + K * 1e-6


def _im2col_brute(x, HH, WW, sh, sw, ph, pw):
    N, C, H, W = x.shape
    Ho, Wo = orc.conv_out(H, W, HH, WW, sh, sw, ph, pw)
    col = np.zeros((C * HH * WW, N * Ho * Wo), np.float32)
    for c in range(C):
        for kh in range(HH):
            for kw in range(WW):
                for n in range(N):
                    for ho in range(Ho):
                        for wo in range(Wo):
                            h, w = ho * sh - ph + kh, wo * sw - pw + kw
                            if 0 <= h < H and 0 <= w < W:
                                col[(c * HH + kh) * WW + kw, (n * Ho + ho) * Wo + wo] = x[n, c, h, w]
    return col


@pytest.mark.parametrize("HH,sh,ph", [(3, 1, 0), (3, 1, 1), (3, 2, 1), (2, 2, 2), (1, 1, 0)])
def test_im2col_brute_force_and_adjoint(HH, sh, ph):
    x = u(2, 3, 6, 5)
    col = orc.im2col(x, HH, HH, sh, sh, ph, ph)
    assert same(col, _im2col_brute(x, HH, HH, sh, sh, ph, ph))
    # col2im is the adjoint of im2col: <im2col(x), c> == <x, col2im(c)>
    c = u(*col.shape)
    back = orc.col2im(c, x.shape, HH, HH, sh, sh, ph, ph)
    lhs = np.dot(col.astype(np.float64).ravel(), c.astype(np.float64).ravel())
    rhs = np.dot(x.astype(np.float64).ravel(), back.astype(np.float64).ravel())
    assert abs(lhs - rhs) < 1e-4 * (1 + abs(lhs))


def test_maxpool_special_values():
    # reference tests/test_ops.py:551-567: -2e30 kept, -inf kept, all-NaN -> -inf
    for v, want in ((-2e30, np.float32(-2e30)), (-np.inf, -np.inf), (np.nan, -np.inf)):
        y = orc.maxpool_fwd(np.full((1, 1, 4, 4), v, np.float32), 2, 2, 2, 2)
        assert np.all(y == want)


def test_maxpool_bwd_first_strict_max_brute():
    x = rng.integers(0, 3, (2, 2, 7, 7)).astype(np.float32)  # many ties
    for p, s in ((2, 2), (3, 2), (2, 1)):
        y = orc.maxpool_fwd(x, p, p, s, s)
        G = u(*y.shape)
        want = np.zeros_like(x)
        for n in range(2):
            for c in range(2):
                for ho in range(y.shape[2]):
                    for wo in range(y.shape[3]):
                        win = x[n, c, ho * s:ho * s + p, wo * s:wo * s + p]
                        k = int(np.argmax(win))  # first maximum in row-major order
                        want[n, c, ho * s + k // p, wo * s + k % p] += G[n, c, ho, wo]
                        assert y[n, c, ho, wo] == win.max()
        assert same(orc.maxpool_bwd(x, G, p, p, s, s), want)


def test_softmax_vs_float64_and_edges():
    x = u(7, 13) * 10
    x[3] += 100.0
    ref = np.exp(x - x.max(1, keepdims=True).astype(np.float64))
    ref /= ref.sum(1, keepdims=True)
    assert np.allclose(orc.softmax_fwd(x), ref, atol=1e-6, rtol=1e-5)
    assert np.all(orc.softmax_fwd(np.full((2, 4), -np.inf, np.float32)) == 0.25)


def _fd(f, x, h=1e-2):
    g = np.zeros(x.size)
    for i in range(x.size):
        xp, xm = x.copy(), x.copy()
        xp.flat[i] += h
        xm.flat[i] -= h
        g[i] = (f(xp) - f(xm)) / (2 * h)
    return g.reshape(x.shape)


def test_conv_backward_vs_finite_differences():
    x, w, b = u(2, 2, 5, 5), u(3, 2, 3, 3), u(3)
    R = u(2, 3, 5, 5).astype(np.float64)
    dx, dw, db = orc.conv2d_bwd(x, w, R.astype(np.float32), 1, 1, 1, 1)
    L = lambda x_, w_, b_: float(np.sum(R * orc.conv2d_fwd(x_, w_, b_, 1, 1, 1, 1)))  # noqa: E731
    assert np.allclose(dx, _fd(lambda t: L(t, w, b), x), atol=2e-3, rtol=1e-3)
    assert np.allclose(dw, _fd(lambda t: L(x, t, b), w), atol=2e-3, rtol=1e-3)
    assert np.allclose(db, _fd(lambda t: L(x, w, t), b), atol=2e-3, rtol=1e-3)


def test_softmax_relu_padones_backward_vs_fd():
    x = u(3, 5)
    x[np.abs(x) < 0.05] = 0.3
    R = u(3, 5).astype(np.float64)
    s = orc.softmax_fwd(x)
    assert np.allclose(orc.softmax_bwd(s, R.astype(np.float32)),
                       _fd(lambda t: float(np.sum(R * orc.softmax_fwd(t))), x), atol=1e-4)
    assert np.allclose(orc.relu_bwd(x, R.astype(np.float32)),
                       _fd(lambda t: float(np.sum(R * orc.relu_fwd(t))), x), atol=1e-4)
    R2 = u(3, 6).astype(np.float64)
    assert np.allclose(orc.padones_bwd(R2.astype(np.float32)),
                       _fd(lambda t: float(np.sum(R2 * orc.padones_fwd(t))), x), atol=1e-4)


def test_mlp_step_vs_finite_differences():
    x, y, Ws = orc.mlp_inputs(B=4, dims=(6, 5, 4, 3), seed=11)
    for W in Ws:
        W[-1] = u(W.shape[1]) * 0.1  # nonzero bias rows
    o = orc.mlp_step(x, y, *Ws)

    def loss(W1, W2, W3):
        return orc.mlp_step(x, y, W1, W2, W3)["loss"]
    num = _fd(lambda t: loss(t, Ws[1], Ws[2]), Ws[0], h=1e-3)
    assert np.allclose(o["dW1"], num, atol=2e-3, rtol=2e-2)
    num = _fd(lambda t: loss(Ws[0], Ws[1], t), Ws[2], h=1e-3)
    assert np.allclose(o["dW3"], num, atol=2e-3, rtol=2e-2)


def test_ce_seed_closed_form():
    p = orc.softmax_fwd(u(6, 10))
    y = np.array([0, 9, 3, 3, 5, 1])
    loss, seed = orc.ce_seed(p, y)
    oh = np.eye(10, dtype=np.float32)[y]
    assert same(seed, (p - oh) / np.float32(6))
    assert abs(loss + np.mean(np.log(p[np.arange(6), y].astype(np.float64)))) < 1e-6


# ---- optimizers of the reference harnesses (SGD-momentum, Adam) ----
# The reference has no compiled optimizer: its harnesses run them in NumPy.
# The oracle writes the NumPy dtype rules out explicitly; these pins check
# them against closed-form trajectories (constant gradient) and against
# NumPy's own promotion of Python-float / NumPy-float64 scalars.

def test_momentum_constant_gradient_closed_form():
    w0 = u(300)
    g = u(300)
    lr, mu, k = 0.1, 0.9, 12
    w, v = w0.copy(), np.zeros_like(w0)
    for _ in range(k):
        orc.momentum_step(w, v, g, lr, mu)
    # v_k = -lr g (1 - mu^k)/(1 - mu);  w_k = w0 + sum_j v_j
    g64 = g.astype(np.float64)
    vk = -lr * g64 * (1 - mu ** k) / (1 - mu)
    wk = w0 + sum(-lr * g64 * (1 - mu ** j) / (1 - mu) for j in range(1, k + 1))
    assert np.abs(v - vk).max() <= 1e-5 * np.abs(vk).max()
    assert np.abs(w - wk).max() <= 1e-5 * np.abs(wk).max()


def test_adam_constant_gradient_closed_form():
    """With a constant g the bias-corrected moments are exactly g and g^2, so
    step t moves w by lr*g*s_t/(|g|*s_t + eps), s_t = sqrt(1-b2^t).  eps is
    chosen comparable to |g| so a misplaced eps or bias correction shows."""
    g = np.concatenate([u(200), np.float32(1e-3) * u(200)])
    w0 = u(400)
    lr, b1, b2, eps = 0.003, 0.9, 0.999, 1e-3
    p, m, v = [w0.copy()], [np.zeros_like(w0)], [np.zeros_like(w0)]
    w = w0.astype(np.float64)
    g64 = g.astype(np.float64)
    for t in range(1, 9):
        orc.adam_step(p, [g], m, v, t, lr, b1, b2, eps)
        s = np.sqrt(1 - b2 ** t)
        w = w - lr * g64 * s / (np.abs(g64) * s + eps)
        assert np.abs(m[0] - g64 * (1 - b1 ** t)).max() <= 1e-6
        assert np.abs(v[0] - g64 ** 2 * (1 - b2 ** t)).max() <= 1e-8
        assert np.abs(p[0] - w).max() <= 2e-6, t


def test_adam_first_step_is_signed_lr():
    """t = 1 with eps -> 0: w1 = w0 - lr*sign(g) (the classic Adam first step)."""
    g = u(500)
    g[np.abs(g) < 1e-3] = 0.5
    w0 = u(500)
    p, m, v = [w0.copy()], [np.zeros_like(w0)], [np.zeros_like(w0)]
    orc.adam_step(p, [g], m, v, 1, lr=0.01, eps=1e-12)
    assert np.abs(p[0] - (w0.astype(np.float64) - 0.01 * np.sign(g))).max() <= 1e-6


def test_optimizer_dtype_rules_match_numpy_promotion():
    """The explicit float32/float64 steps of the oracle equal what NumPy does
    when the harness's expressions mix float32 arrays with a Python float
    (weak: rounded to float32) and with a NumPy float64 scalar (strong:
    promotes the array expression to float64, rounded by the in-place -=)."""
    w, v, g = u(1000), u(1000), u(1000)
    w1, v1 = w.copy(), v.copy()
    orc.momentum_step(w1, v1, g, 0.1, 0.9)
    v2 = 0.9 * v - 0.1 * g
    w2 = w.copy()
    w2 += v2
    assert v2.dtype == np.float32
    assert np.array_equal(v1, v2) and np.array_equal(w1, w2)

    p, m, vv = u(1000), u(1000) * np.float32(0.1), np.abs(u(1000)) * np.float32(0.01)
    P1, M1, V1 = [p.copy()], [m.copy()], [vv.copy()]
    orc.adam_step(P1, [g], M1, V1, 3)
    lr_t = 0.003 * (np.sqrt(1.0 - 0.999 ** 3) / (1.0 - 0.9 ** 3))
    assert isinstance(lr_t, np.float64)
    m2 = 0.9 * m + (1.0 - 0.9) * g
    v3 = 0.999 * vv + (1.0 - 0.999) * (g * g)
    step = lr_t * m2 / (np.sqrt(v3) + 1e-8)
    assert m2.dtype == np.float32 and step.dtype == np.float64
    p2 = p.copy()
    p2 -= step
    assert np.array_equal(M1[0], m2) and np.array_equal(V1[0], v3)
    assert np.array_equal(P1[0], p2)


# ---- dataset formats and normalisation ----

def _write_idx(path, arr, gz):
    import gzip
    import struct
    arr = np.ascontiguousarray(arr, np.uint8)
    raw = struct.pack(">BBBB", 0, 0, 0x08, arr.ndim) + struct.pack(">" + "I" * arr.ndim, *arr.shape)
    raw += arr.tobytes()
    with (gzip.open(path, "wb") if gz else open(path, "wb")) as f:
        f.write(raw)


@pytest.mark.parametrize("gz", [False, True])
def test_idx_reader_and_probe(tmp_path, gz):
    """the oracle reader and the library's host-side header parser agree with
    a file written from the format's definition"""
    import ctypes
    import tinytorch_amd
    img = rng.integers(0, 256, (7, 28, 28), dtype=np.uint8)
    p = str(tmp_path / ("img.idx.gz" if gz else "img.idx"))
    _write_idx(p, img, gz)
    assert np.array_equal(orc.read_idx(p), img)
    L = tinytorch_amd.lib()
    nd = ctypes.c_int()
    dims = (ctypes.c_long * 8)()
    assert L.tt_idx_probe(p.encode(), ctypes.byref(nd), dims) == 0
    assert tuple(dims[: nd.value]) == (7, 28, 28)
    bad = str(tmp_path / "bad.idx")
    with open(bad, "wb") as f:
        f.write(bytes([0, 0, 0x0D, 1, 0, 0, 0, 4]) + b"\0" * 16)  # float32 idx: rejected
    assert L.tt_idx_probe(bad.encode(), ctypes.byref(nd), dims) != 0
    assert L.tt_idx_probe(str(tmp_path / "missing").encode(), ctypes.byref(nd), dims) != 0


def test_cifar_bin_reader(tmp_path):
    ims = [rng.integers(0, 256, (n, 3, 32, 32), dtype=np.uint8) for n in (3, 5)]
    labs = [rng.integers(0, 10, n).astype(np.int32) for n in (3, 5)]
    paths = []
    for i, (im, lb) in enumerate(zip(ims, labs)):
        p = str(tmp_path / f"b{i}.bin")
        with open(p, "wb") as f:
            for k in range(len(lb)):
                f.write(bytes([lb[k]]) + im[k].tobytes())  # label byte, then R, G, B planes
        paths.append(p)
    x, y = orc.read_cifar_bin(paths)
    assert np.array_equal(x, np.concatenate(ims)) and np.array_equal(y, np.concatenate(labs))


def test_normalize_matches_numpy_harness_forms_and_float64():
    x = np.arange(256, dtype=np.uint8).reshape(1, 1, 16, 16)
    # MNIST form: Python-float mean/std against a float32 array
    got = orc.normalize_u8(x, [0.1307], [0.3081])
    harness = ((x.astype(np.float32) / 255.0) - 0.1307) / 0.3081
    assert harness.dtype == np.float32 and np.array_equal(got, harness)
    # CIFAR form: float32 (1, 3, 1, 1) arrays
    x3 = rng.integers(0, 256, (4, 3, 8, 8), dtype=np.uint8)
    mean = np.array([0.4914, 0.4822, 0.4465], dtype=np.float32).reshape(1, 3, 1, 1)
    std = np.array([0.2023, 0.1994, 0.2010], dtype=np.float32).reshape(1, 3, 1, 1)
    got3 = orc.normalize_u8(x3, mean.ravel(), std.ravel())
    assert np.array_equal(got3, (x3.astype(np.float32) / 255.0 - mean) / std)
    # and within float32 rounding of the exact value
    exact = (x3 / 255.0 - mean.astype(np.float64)) / std.astype(np.float64)
    assert np.abs(got3 - exact).max() <= 4e-7 * np.abs(exact).max()
