"""GPU kernels vs the oracle, through the device-level C ABI (include/tt_hip.h).

Bars:
  * index / selection / copy work -- im2col, col2im, maxpool fwd/bwd,
    avgpool, relu, padones, softmax backward -- bit-exact;
  * GEMMs: max|C - C_oracle| / (sqrt(K) * max|A| * max|B|) <= 1e-4 and
    max|C - C_oracle| / max|C_oracle| <= 1e-4;
  * softmax forward (device expf vs libm expf) and the bias-grad reduction
    (tree vs serial order): max relative error <= 1e-5.
"""
import ctypes

import numpy as np
import pytest

import orc
from tinytorch_amd.hip import DevBuf, check, sync

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(99)

GEMM_TOL = 1e-4


def u(*s):
    return rng.uniform(-1, 1, s).astype(np.float32)


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def gemm_err(C, ref, K, amax, bmax):
    ref = np.asarray(ref, np.float64)
    d = np.abs(np.asarray(C, np.float64) - ref).max() if C.size else 0.0
    norm = d / (np.sqrt(max(K, 1)) * max(amax, 1e-30) * max(bmax, 1e-30))
    rel = d / max(np.abs(ref).max(), 1e-30) if C.size else 0.0
    return norm, rel


def run_gemm(tlib, M, N, K, ta, tb, A, B):
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(M * N)
    lda = A.shape[1]
    ldb = B.shape[1]
    print(f"gemm M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    check(tlib.tt_k_gemm(M, N, K, dA.ptr, lda, ta, dB.ptr, ldb, tb, dC.ptr, N), "tt_k_gemm")
    return dC.to_np((M, N))


SHAPES = [(1, 1, 1), (3, 4, 5), (17, 13, 5), (5, 300, 3), (9, 33, 256), (64, 16, 512),
          (128, 128, 32), (100, 70, 33), (1000, 1003, 997), (256, 512, 785), (256, 10, 257),
          (513, 65, 1024), (31, 2000, 7), (100, 7, 3000)]


def test_gemm_skinny_split_leading_dims(tlib):
    """A skinny GEMM over a long K (the 16x16 split-K tiles) with leading
    dimensions wider than the rows: A (lda = K + 4), B (ldb = N + 3) and C
    (ldc = N + 1) read and written only where the matrix is; the padding of
    C stays as it was."""
    M, N, K = 70, 9, 2500
    A = u(M, K + 4)
    B = u(K, N + 3)
    C0 = np.full((M, N + 1), 7.0, np.float32)
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf.from_np(C0)
    print("gemm skinny split ld", M, N, K, flush=True)
    check(tlib.tt_k_gemm(M, N, K, dA.ptr, K + 4, 0, dB.ptr, N + 3, 0, dC.ptr, N + 1), "gemm")
    C = dC.to_np((M, N + 1))
    ref = orc.sgemm(A[:, :K], B[:, :N])
    norm, rel = gemm_err(C[:, :N], ref, K, np.abs(A).max(), np.abs(B).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)
    assert np.all(C[:, N] == 7.0)


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_nn_vs_oracle(tlib, M, N, K):
    A, B = u(M, K), u(K, N)
    C = run_gemm(tlib, M, N, K, 0, 0, A, B)
    ref = orc.sgemm(A, B)
    norm, rel = gemm_err(C, ref, K, np.abs(A).max(), np.abs(B).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_nt_vs_oracle(tlib, M, N, K):
    """dA = dC * B^T: opA = G (M x K), opB stored N x K (matmul_nt)."""
    G, B = rng.standard_normal((M, K)).astype(np.float32), u(N, K)
    C = run_gemm(tlib, M, N, K, 0, 1, G, B)
    ref = orc.matmul_nt(G, B)
    norm, rel = gemm_err(C, ref, K, np.abs(G).max(), np.abs(B).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_tn_vs_oracle(tlib, M, N, K):
    """dB = A^T * dC: opA stored K x M, opB = G (K x N) (matmul_tn)."""
    A, G = u(K, M), rng.standard_normal((K, N)).astype(np.float32)
    C = run_gemm(tlib, M, N, K, 1, 0, A, G)
    ref = orc.matmul_tn(A, G)
    norm, rel = gemm_err(C, ref, K, np.abs(A).max(), np.abs(G).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


@pytest.mark.parametrize("M,N,K", [(7, 9, 11), (130, 70, 300)])
def test_gemm_tt_vs_float64(tlib, M, N, K):
    A, B = u(K, M), u(N, K)
    C = run_gemm(tlib, M, N, K, 1, 1, A, B)
    ref = A.T.astype(np.float64) @ B.T.astype(np.float64)
    norm, rel = gemm_err(C, ref, K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL


def test_gemm_k_zero_gives_zeros(tlib):
    dA, dB, dC = DevBuf(4), DevBuf(4), DevBuf(6)
    dC.fill(7.0)
    check(tlib.tt_k_gemm(2, 3, 0, dA.ptr, 1, 0, dB.ptr, 3, 0, dC.ptr, 3), "gemm K=0")
    assert np.all(dC.to_np() == 0.0)


def test_gemm_rejects_bad_args(tlib):
    d = DevBuf(4)
    assert tlib.tt_k_gemm(-1, 2, 2, d.ptr, 2, 0, d.ptr, 2, 0, d.ptr, 2) != 0
    assert tlib.tt_k_gemm(2, 2, 2, None, 2, 0, d.ptr, 2, 0, d.ptr, 2) != 0


CONV_CASES = [  # (N, C, H, W, F, HH, WW, sh, sw, ph, pw)
    (2, 3, 7, 7, 4, 3, 3, 1, 1, 1, 1), (2, 3, 7, 7, 4, 3, 3, 2, 2, 0, 0),
    (3, 4, 9, 8, 5, 3, 2, 2, 1, 2, 1), (1, 1, 5, 5, 1, 1, 1, 1, 1, 0, 0),
    (4, 32, 16, 16, 64, 3, 3, 1, 1, 1, 1), (8, 3, 32, 32, 32, 3, 3, 1, 1, 1, 1),
    (2, 5, 6, 6, 3, 5, 5, 1, 1, 2, 2),
    # strided planes that fit the LDS-staged col2im (Ho*Wo % 4 == 0), 4-pixel and 1-pixel lanes
    (2, 3, 8, 8, 4, 3, 3, 2, 2, 1, 1), (2, 2, 8, 14, 3, 2, 2, 2, 2, 0, 0),
]


def conv_dims(N, C, H, W, F, HH, WW, sh, sw, ph, pw):
    Ho, Wo = orc.conv_out(H, W, HH, WW, sh, sw, ph, pw)
    return Ho, Wo, C * HH * WW, N * Ho * Wo


@pytest.mark.parametrize("case", CONV_CASES)
def test_im2col_col2im_bitexact(tlib, case):
    N, C, H, W, F, HH, WW, sh, sw, ph, pw = case
    Ho, Wo, Kc, Ncol = conv_dims(*case)
    x = u(N, C, H, W)
    dx, dcol = DevBuf.from_np(x), DevBuf(Kc * Ncol)
    print("im2col", case, flush=True)
    check(tlib.tt_k_im2col(dx.ptr, dcol.ptr, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo), "im2col")
    assert bits_equal(dcol.to_np((Kc, Ncol)), orc.im2col(x, HH, WW, sh, sw, ph, pw))
    col = u(Kc, Ncol)
    dc, dimg = DevBuf.from_np(col), DevBuf(x.size)
    print("col2im", case, flush=True)
    check(tlib.tt_k_col2im(dc.ptr, dimg.ptr, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo), "col2im")
    assert bits_equal(dimg.to_np(x.shape), orc.col2im(col, x.shape, HH, WW, sh, sw, ph, pw))


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_gemms_vs_oracle(tlib, case):
    N, C, H, W, F, HH, WW, sh, sw, ph, pw = case
    Ho, Wo, Kc, Ncol = conv_dims(*case)
    x, w, b = u(N, C, H, W), u(F, C, HH, WW), u(F)
    col = orc.im2col(x, HH, WW, sh, sw, ph, pw)
    dcol, dw, db, dout = DevBuf.from_np(col), DevBuf.from_np(w), DevBuf.from_np(b), DevBuf(N * F * Ho * Wo)
    print("conv_fwd", case, flush=True)
    check(tlib.tt_k_conv_fwd(F, Kc, Ncol, Ho * Wo, dw.ptr, dcol.ptr, db.ptr, dout.ptr), "conv_fwd")
    ref = orc.conv2d_fwd(x, w, b, sh, sw, ph, pw)
    norm, rel = gemm_err(dout.to_np(ref.shape) - b[None, :, None, None],
                         ref - b[None, :, None, None], Kc, np.abs(w).max(), np.abs(x).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL
    g = rng.standard_normal((N, F, Ho, Wo)).astype(np.float32)
    rdx, rdw, _ = orc.conv2d_bwd(x, w, g, sh, sw, ph, pw, need_db=False)
    dg, ddw = DevBuf.from_np(g), DevBuf(w.size)
    print("conv_dw", case, flush=True)
    check(tlib.tt_k_conv_dw(F, Kc, Ncol, Ho * Wo, dg.ptr, dcol.ptr, ddw.ptr), "conv_dw")
    norm, rel = gemm_err(ddw.to_np(w.shape), rdw, Ncol, np.abs(g).max(), np.abs(x).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL
    ddc = DevBuf(Kc * Ncol)
    print("conv_dcol", case, flush=True)
    check(tlib.tt_k_conv_dcol(F, Kc, Ncol, Ho * Wo, dw.ptr, dg.ptr, ddc.ptr), "conv_dcol")
    gp = g.transpose(1, 0, 2, 3).reshape(F, Ncol)
    ref_dcol = orc.sgemm(np.ascontiguousarray(w.reshape(F, Kc).T), gp)
    norm, rel = gemm_err(ddc.to_np((Kc, Ncol)), ref_dcol, F, np.abs(w).max(), np.abs(g).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL
    # end to end dX = col2im(dcol) vs the oracle's conv backward
    dimg = DevBuf(x.size)
    check(tlib.tt_k_col2im(ddc.ptr, dimg.ptr, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo), "col2im")
    got = dimg.to_np(x.shape)
    assert np.abs(got - rdx).max() <= GEMM_TOL * max(np.abs(rdx).max(), 1e-30) * 4


POOL_CASES = [(2, 2), (3, 2), (2, 1), (3, 3), (1, 1)]


def pool_input(shape):
    x = rng.integers(-3, 3, shape).astype(np.float32) * 0.5  # plenty of ties
    x[0, 0, :3, :3] = -np.inf
    x[0, 1, :3, :3] = np.nan
    x[-1, -1, 0, 1] = np.nan
    x[0, 2 % shape[1], 0, 0] = -2e30
    return x


@pytest.mark.parametrize("p,s", POOL_CASES)
def test_maxpool_bitexact(tlib, p, s):
    x = pool_input((3, 4, 9, 8))
    N, C, H, W = x.shape
    Ho, Wo = orc.pool_out(H, W, p, p, s, s)
    dx_, dy = DevBuf.from_np(x), DevBuf(N * C * Ho * Wo)
    print("maxpool", p, s, flush=True)
    check(tlib.tt_k_maxpool_fwd(dx_.ptr, dy.ptr, N, C, H, W, p, p, s, s, Ho, Wo), "maxpool_fwd")
    assert bits_equal(dy.to_np((N, C, Ho, Wo)), orc.maxpool_fwd(x, p, p, s, s))
    g = u(N, C, Ho, Wo)
    g[0, 0, 0, 0] = -0.0
    dg, dgx = DevBuf.from_np(g), DevBuf(x.size)
    check(tlib.tt_k_maxpool_bwd(dx_.ptr, dg.ptr, dgx.ptr, N, C, H, W, p, p, s, s, Ho, Wo), "maxpool_bwd")
    assert bits_equal(dgx.to_np(x.shape), orc.maxpool_bwd(x, g, p, p, s, s))


CONFIG4_POOLS = [(128, 32, 32, 32), (128, 64, 16, 16)]


@pytest.mark.parametrize("shape", CONFIG4_POOLS)
def test_maxpool2x2_config4_bitexact(tlib, shape):
    """The 2x2/s2 fast kernels at the CNN config's activation shapes: forward
    values and backward argmax routing bit-exact against the oracle (ties,
    NaN, -Inf, -2e30 and -0.0 gradients included)."""
    x = pool_input(shape)
    N, C, H, W = shape
    Ho, Wo = H // 2, W // 2
    dx_, dy = DevBuf.from_np(x), DevBuf(N * C * Ho * Wo)
    print("maxpool config4", shape, flush=True)
    check(tlib.tt_k_maxpool_fwd(dx_.ptr, dy.ptr, N, C, H, W, 2, 2, 2, 2, Ho, Wo), "maxpool_fwd")
    assert bits_equal(dy.to_np((N, C, Ho, Wo)), orc.maxpool_fwd(x, 2, 2, 2, 2))
    g = u(N, C, Ho, Wo)
    g[0, 0, 0, 0] = -0.0
    dg, dgx = DevBuf.from_np(g), DevBuf(x.size)
    check(tlib.tt_k_maxpool_bwd(dx_.ptr, dg.ptr, dgx.ptr, N, C, H, W, 2, 2, 2, 2, Ho, Wo),
          "maxpool_bwd")
    assert bits_equal(dgx.to_np(x.shape), orc.maxpool_bwd(x, g, 2, 2, 2, 2))


@pytest.mark.parametrize("shape", [(3, 4, 9, 8), (2, 3, 8, 12)] + CONFIG4_POOLS)
def test_maxpool_relu_fused_bitexact(tlib, shape):
    """The fused 2x2 pool + relu backward against the reference's two steps:
    the pool's input r is relu(x); dr = maxpool backward, dx = relu backward
    of dr evaluated on x (NaN, -0.0 and exact zeros in x; odd H leaves a row
    the pool does not cover)."""
    x = pool_input(shape)
    x[0, 0, 4, :4] = [0.0, -0.0, 1e-30, -1e-30]
    N, C, H, W = shape
    Ho, Wo = orc.pool_out(H, W, 2, 2, 2, 2)
    r = orc.relu_fwd(x)
    g = u(N, C, Ho, Wo)
    g[0, 0, 0, 0] = -0.0
    dr_ref = orc.maxpool_bwd(r, g, 2, 2, 2, 2)
    dx_ref = orc.relu_bwd(x, dr_ref)
    dr_, dg, ddr, ddx = DevBuf.from_np(r), DevBuf.from_np(g), DevBuf(x.size), DevBuf(x.size)
    print("maxpool+relu bwd", shape, flush=True)
    check(tlib.tt_k_maxpool2x2_relu_bwd(dr_.ptr, dg.ptr, ddr.ptr, ddx.ptr, N, C, H, W, Ho, Wo),
          "maxpool2x2_relu_bwd")
    assert bits_equal(ddr.to_np(shape), dr_ref)
    assert bits_equal(ddx.to_np(shape), dx_ref)
    # from the relu's input (the relu taken on load), and without dr
    dxp, ddr2, ddx2 = DevBuf.from_np(x), DevBuf(x.size), DevBuf(x.size)
    check(tlib.tt_k_maxpool2x2_prerelu_bwd(dxp.ptr, dg.ptr, ddr2.ptr, ddx2.ptr, N, C, H, W, Ho, Wo),
          "maxpool2x2_prerelu_bwd")
    assert bits_equal(ddr2.to_np(shape), dr_ref)
    assert bits_equal(ddx2.to_np(shape), dx_ref)
    ddx3 = DevBuf(x.size)
    check(tlib.tt_k_maxpool2x2_prerelu_bwd(dxp.ptr, dg.ptr, None, ddx3.ptr, N, C, H, W, Ho, Wo),
          "maxpool2x2_prerelu_bwd dx only")
    assert bits_equal(ddx3.to_np(shape), dx_ref)


@pytest.mark.parametrize("p,s", POOL_CASES)
def test_avgpool_bitexact(tlib, p, s):
    x = u(2, 3, 9, 8)
    N, C, H, W = x.shape
    Ho, Wo = orc.pool_out(H, W, p, p, s, s)
    dx_, dy = DevBuf.from_np(x), DevBuf(N * C * Ho * Wo)
    check(tlib.tt_k_avgpool_fwd(dx_.ptr, dy.ptr, N, C, H, W, p, p, s, s, Ho, Wo), "avgpool_fwd")
    assert bits_equal(dy.to_np((N, C, Ho, Wo)), orc.avgpool_fwd(x, p, p, s, s))
    g = u(N, C, Ho, Wo)
    dg, dgx = DevBuf.from_np(g), DevBuf(x.size)
    check(tlib.tt_k_avgpool_bwd(dg.ptr, dgx.ptr, N, C, H, W, p, p, s, s, Ho, Wo), "avgpool_bwd")
    assert bits_equal(dgx.to_np(x.shape), orc.avgpool_bwd(g, x.shape, p, p, s, s))


@pytest.mark.parametrize("n", [0, 1, 3, 4, 1001, 1 << 20])
def test_relu_bitexact(tlib, n):
    x = rng.standard_normal(n).astype(np.float32)
    if n >= 4:
        x[:4] = [np.nan, np.inf, -np.inf, -0.0]
    g = rng.standard_normal(n).astype(np.float32)
    dx_, dg, dy, ddx = DevBuf.from_np(x), DevBuf.from_np(g), DevBuf(n), DevBuf(n)
    check(tlib.tt_k_relu_fwd(dx_.ptr, dy.ptr, n), "relu_fwd")
    check(tlib.tt_k_relu_bwd(dx_.ptr, dg.ptr, ddx.ptr, n), "relu_bwd")
    assert bits_equal(dy.to_np(), orc.relu_fwd(x))
    assert bits_equal(ddx.to_np(), orc.relu_bwd(x, g))


@pytest.mark.parametrize("rows,cols", [(1, 1), (6, 10), (128, 10), (5, 64), (7, 65), (3, 1000)])
def test_softmax(tlib, rows, cols):
    x = (u(rows, cols) * 8).astype(np.float32)
    if rows > 2:
        x[1] = -np.inf
        x[2] += 100.0
    dx_, dy = DevBuf.from_np(x), DevBuf(x.size)
    check(tlib.tt_k_softmax_fwd(dx_.ptr, dy.ptr, rows, cols), "softmax_fwd")
    y = dy.to_np(x.shape)
    ref = orc.softmax_fwd(x)
    assert np.abs(y - ref).max() <= 1e-5 * max(np.abs(ref).max(), 1e-30)
    if rows > 2:
        assert np.all(y[1] == np.float32(1.0) / np.float32(cols))
    g = u(rows, cols)
    s = ref
    ds, dg, ddx = DevBuf.from_np(s), DevBuf.from_np(g), DevBuf(x.size)
    check(tlib.tt_k_softmax_bwd(ds.ptr, dg.ptr, ddx.ptr, rows, cols), "softmax_bwd")
    got = ddx.to_np(x.shape)
    want = orc.softmax_bwd(s, g)
    if cols <= 64:  # one row per lane keeps the reference's serial dot order
        assert bits_equal(got, want)
    else:
        assert np.abs(got - want).max() <= 1e-5 * max(np.abs(want).max(), 1e-30)


@pytest.mark.parametrize("M,K", [(1, 1), (256, 784), (128, 4096), (3, 5)])
def test_padones_bitexact(tlib, M, K):
    x = u(M, K)
    dx_, dy = DevBuf.from_np(x), DevBuf(M * (K + 1))
    check(tlib.tt_k_padones_fwd(dx_.ptr, dy.ptr, M, K), "padones_fwd")
    assert bits_equal(dy.to_np((M, K + 1)), orc.padones_fwd(x))
    g = u(M, K + 1)
    dg, ddx = DevBuf.from_np(g), DevBuf(M * K)
    check(tlib.tt_k_padones_bwd(dg.ptr, ddx.ptr, M, K), "padones_bwd")
    assert bits_equal(ddx.to_np((M, K)), orc.padones_bwd(g))


@pytest.mark.parametrize("M,K", [(1, 1), (256, 512), (3, 1030)])
def test_padones_relu_fused_bitexact(tlib, M, K):
    """The fused padones + relu backward against the reference's two steps
    (relu backward evaluated on the relu's input x: NaN, -0.0, exact zeros)."""
    x = rng.standard_normal((M, K)).astype(np.float32)
    x.flat[: min(4, x.size)] = [0.0, -0.0, np.nan, 1e-38][: min(4, x.size)]
    r = orc.relu_fwd(x)
    g = u(M, K + 1)
    dr_ref = orc.padones_bwd(g)
    dr_, dg, ddr, ddx = DevBuf.from_np(r), DevBuf.from_np(g), DevBuf(M * K), DevBuf(M * K)
    check(tlib.tt_k_padones_relu_bwd(dg.ptr, dr_.ptr, ddr.ptr, ddx.ptr, M, K), "padones_relu_bwd")
    assert bits_equal(ddr.to_np((M, K)), dr_ref)
    assert bits_equal(ddx.to_np((M, K)), orc.relu_bwd(x, dr_ref))


@pytest.mark.parametrize("N,F,HW", [(1, 1, 1), (2, 4, 49), (128, 32, 1024), (128, 64, 256),
                                    (64, 5000, 3), (128, 3, 100)])
def test_bias_grad(tlib, N, F, HW):
    """Two deterministic stages (partials, then their in-order sum): a second
    call gives the same bits; F beyond one partial a filter, tiny HW."""
    g = rng.standard_normal((N, F, HW)).astype(np.float32)
    dg, db = DevBuf.from_np(g), DevBuf(F)
    check(tlib.tt_k_bias_grad(dg.ptr, db.ptr, N, F, HW), "bias_grad")
    first = db.to_np()
    check(tlib.tt_k_bias_grad(dg.ptr, db.ptr, N, F, HW), "bias_grad again")
    assert bits_equal(db.to_np(), first)
    ref = orc.bias_grad(g)
    exact = g.astype(np.float64).sum(axis=(0, 2))
    got = db.to_np()
    # serial fp32 (the reference) and tree fp32 (here) both sit near the exact sum
    scale = np.abs(g).sum(axis=(0, 2)).max()
    assert np.abs(got - exact).max() <= 1e-5 * scale + 1e-6
    assert np.abs(got - ref).max() <= 2e-5 * scale + 1e-6


def test_softmax_ce_closed_form(tlib):
    rows, cols = 128, 10
    x = (u(rows, cols) * 4).astype(np.float32)
    y = rng.integers(0, cols, rows).astype(np.int32)
    dx_, dlab = DevBuf.from_np(x), DevBuf.from_np(y)
    dp, dl, ds = DevBuf(x.size), DevBuf(rows), DevBuf(x.size)
    check(tlib.tt_k_softmax_ce(dx_.ptr, dlab.ptr, dp.ptr, dl.ptr, ds.ptr, rows, cols,
                               ctypes.c_float(1.0 / rows)), "softmax_ce")
    p = orc.softmax_fwd(x)
    loss, seed = orc.ce_seed(p, y)
    assert np.abs(dp.to_np(x.shape) - p).max() <= 1e-6
    assert np.abs(ds.to_np(x.shape) - seed).max() <= 1e-7
    assert abs(float(dl.to_np().astype(np.float64).mean()) - loss) <= 1e-5


def test_copy_fill_add_sgd(tlib):
    n = 12345
    a, b = u(n), u(n)
    da, db = DevBuf.from_np(a), DevBuf.from_np(b)
    check(tlib.tt_k_add_inplace(da.ptr, db.ptr, n), "add_inplace")
    assert bits_equal(da.to_np(), a + b)
    check(tlib.tt_k_copy(da.ptr, db.ptr, n), "copy")
    assert bits_equal(da.to_np(), b)
    check(tlib.tt_k_fill(da.ptr, n, ctypes.c_float(2.5)), "fill")
    assert np.all(da.to_np() == 2.5)
    sync()


@pytest.mark.parametrize("rows,cols", [(1, 3), (128, 10), (1000, 17), (8192, 10)])
def test_softmax_ce_mean_one_launch(tlib, rows, cols):
    x = (u(rows, cols) * 4).astype(np.float32)
    y = rng.integers(0, cols, rows).astype(np.int32)
    dx_, dlab = DevBuf.from_np(x), DevBuf.from_np(y)
    dp, dl, ds = DevBuf(x.size), DevBuf(1), DevBuf(x.size)
    check(tlib.tt_k_softmax_ce_mean(dx_.ptr, dlab.ptr, dp.ptr, dl.ptr, ds.ptr, rows, cols,
                                    ctypes.c_float(1.0 / rows)), "softmax_ce_mean")
    p = orc.softmax_fwd(x)
    loss, seed = orc.ce_seed(p, y)
    assert np.abs(dp.to_np(x.shape) - p).max() <= 1e-6
    assert np.abs(ds.to_np(x.shape) - seed).max() <= 1e-7
    assert abs(float(dl.to_np()[0]) - loss) <= 1e-5 * max(1.0, loss)
    assert tlib.tt_k_softmax_ce_mean(dx_.ptr, dlab.ptr, dp.ptr, dl.ptr, ds.ptr, 8193, cols,
                                     ctypes.c_float(1.0)) != 0  # above the one-workgroup limit


def test_scale_by_dev_and_sgd_multi(tlib):
    x = u(1000)
    s = np.array([-1.75], np.float32)
    dx_, ds, dy = DevBuf.from_np(x), DevBuf.from_np(s), DevBuf(1000)
    check(tlib.tt_k_scale_by_dev(dx_.ptr, ds.ptr, dy.ptr, 1000), "scale_by_dev")
    assert bits_equal(dy.to_np(), x * np.float32(-1.75))
    sizes = [1, 7, 4096, 100003]
    ws = [u(n) for n in sizes]
    gs = [u(n) for n in sizes]
    dws = [DevBuf.from_np(w) for w in ws]
    dgs = [DevBuf.from_np(g) for g in gs]
    W = (ctypes.c_void_p * 4)(*[d.ptr for d in dws])
    G = (ctypes.c_void_p * 4)(*[d.ptr for d in dgs])
    Nn = (ctypes.c_long * 4)(*sizes)
    check(tlib.tt_k_sgd_multi(W, G, Nn, 4, ctypes.c_float(0.1)), "sgd_multi")
    for w, g, d in zip(ws, gs, dws):
        assert np.abs(d.to_np() - (w - np.float32(0.1) * g)).max() <= 1e-7
    assert tlib.tt_k_sgd_multi(W, G, Nn, 17, ctypes.c_float(0.1)) != 0


TILE_IDS = range(7)  # 128x128, 128x64, 64x64, 32x256, 64x256, 256x256, 256x128


@pytest.fixture
def forced_config(tlib):
    yield lambda t, s: check(tlib.tth_gemm_config(t, s), "tth_gemm_config")
    tlib.tth_gemm_config(-1, -1)


@pytest.mark.parametrize("tile", TILE_IDS)
@pytest.mark.parametrize("splits", [1, 3])
def test_every_tile_and_split_all_layouts(tlib, forced_config, tile, splits):
    """Every tile configuration x split count, all four layouts, ragged edges
    in M, N and K (so interior fast loads and bounds-checked edge loads both
    run), against the oracle GEMM family."""
    forced_config(tile, splits)
    M, N, K = 300, 270, 161
    A, B = u(M, K), u(K, N)
    G = rng.standard_normal((M, N)).astype(np.float32)
    for ta, tb, a, b, ref, k, am, bm in (
            (0, 0, A, B, orc.sgemm(A, B), K, A, B),
            (0, 1, G, B, orc.matmul_nt(G, B), N, G, B),
            (1, 0, A, G, orc.matmul_tn(A, G), M, A, G),
            (1, 1, np.ascontiguousarray(A.T), np.ascontiguousarray(B.T), orc.sgemm(A, B), K, A, B)):
        Mo, No = ref.shape
        C = run_gemm(tlib, Mo, No, k, ta, tb, a, b)
        norm, rel = gemm_err(C, ref, k, np.abs(am).max(), np.abs(bm).max())
        assert norm <= GEMM_TOL and rel <= GEMM_TOL, (tile, splits, ta, tb, norm, rel)


@pytest.mark.parametrize("tile", TILE_IDS)
def test_every_tile_conv_gemms(tlib, forced_config, tile):
    forced_config(tile, 2)
    N, C, H, W, F = 3, 5, 10, 9, 6
    x, w, b = u(N, C, H, W), u(F, C, 3, 3), u(F)
    Ho, Wo, Kc, Ncol = conv_dims(N, C, H, W, F, 3, 3, 1, 1, 1, 1)
    col = orc.im2col(x, 3, 3, 1, 1, 1, 1)
    dcol, dw, db = DevBuf.from_np(col), DevBuf.from_np(w), DevBuf.from_np(b)
    dout = DevBuf(N * F * Ho * Wo)
    check(tlib.tt_k_conv_fwd(F, Kc, Ncol, Ho * Wo, dw.ptr, dcol.ptr, db.ptr, dout.ptr), "conv_fwd")
    ref = orc.conv2d_fwd(x, w, b, 1, 1, 1, 1)
    assert np.abs(dout.to_np(ref.shape) - ref).max() <= GEMM_TOL * np.sqrt(Kc)
    g = rng.standard_normal((N, F, Ho, Wo)).astype(np.float32)
    rdx, rdw, _ = orc.conv2d_bwd(x, w, g, 1, 1, 1, 1, need_db=False)
    dg, ddw, ddc = DevBuf.from_np(g), DevBuf(w.size), DevBuf(Kc * Ncol)
    check(tlib.tt_k_conv_dw(F, Kc, Ncol, Ho * Wo, dg.ptr, dcol.ptr, ddw.ptr), "conv_dw")
    norm, rel = gemm_err(ddw.to_np(w.shape), rdw, Ncol, np.abs(g).max(), 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL
    check(tlib.tt_k_conv_dcol(F, Kc, Ncol, Ho * Wo, dw.ptr, dg.ptr, ddc.ptr), "conv_dcol")
    gp = g.transpose(1, 0, 2, 3).reshape(F, Ncol)
    ref_dcol = orc.sgemm(np.ascontiguousarray(w.reshape(F, Kc).T), gp)
    norm, rel = gemm_err(ddc.to_np((Kc, Ncol)), ref_dcol, F, 1.0, np.abs(g).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_dw_bias_fused(tlib, case):
    """dW and db from one GEMM against [col; ones] vs the oracle's dW and
    serial bias sum (reference src/autograd.c:467-507)."""
    N, C, H, W, F, HH, WW, sh, sw, ph, pw = case
    Ho, Wo, Kc, Ncol = conv_dims(*case)
    x = u(N, C, H, W)
    dx_, dcol = DevBuf.from_np(x), DevBuf((Kc + 1) * Ncol)
    check(tlib.tt_k_im2col_ones(dx_.ptr, dcol.ptr, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo), "im2col_ones")
    col1 = dcol.to_np((Kc + 1, Ncol))
    assert bits_equal(col1[:Kc], orc.im2col(x, HH, WW, sh, sw, ph, pw)) and np.all(col1[Kc] == 1.0)
    g = rng.standard_normal((N, F, Ho, Wo)).astype(np.float32)
    _, rdw, rdb = orc.conv2d_bwd(x, u(F, C, HH, WW), g, sh, sw, ph, pw, need_dx=False)
    dg, ddw, ddb = DevBuf.from_np(g), DevBuf(F * Kc), DevBuf(F)
    check(tlib.tt_k_conv_dw_bias(F, Kc, Ncol, Ho * Wo, dg.ptr, dcol.ptr, ddw.ptr, ddb.ptr), "conv_dw_bias")
    norm, rel = gemm_err(ddw.to_np(rdw.shape), rdw, Ncol, np.abs(g).max(), np.abs(x).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL
    db = ddb.to_np()
    assert np.abs(db - rdb).max() <= 1e-5 * np.abs(g).sum(axis=(0, 2, 3)).max() + 1e-6


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K,splits", [(512, 768, 1056, 1), (512, 768, 1056, 3),
                                          (256, 256, 32, 1), (768, 512, 4096, 4)])
def test_gemm_direct_lds_kernel(tlib, M, N, K, splits, ta, tb):
    """The direct-to-LDS 256x256 kernel (forced: tile 5) in every
    transposition layout against float64, and bit for bit against the
    register-staged 256x256 kernel, which sums in the same order; with
    split-K the deterministic reduction follows."""
    A = u(K, M) if ta else u(M, K)
    B = u(N, K) if tb else u(K, N)
    try:
        tlib.tth_gemm_config(5, splits)
        C = run_gemm(tlib, M, N, K, ta, tb, A, B)
        tlib.tth_gemm_direct(0)
        C_staged = run_gemm(tlib, M, N, K, ta, tb, A, B)
    finally:
        tlib.tth_gemm_direct(1)
        tlib.tth_gemm_config(-1, -1)
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    norm, rel = gemm_err(C, ref, K, np.abs(A).max(), np.abs(B).max())
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)
    assert bits_equal(C, C_staged)


# Shapes for the 64x64 direct-load kernel (16-byte aligned rows, K and the
# m/n-contiguous extents multiples of 4): edge tiles in M and N, K tails
# inside a 64-k tile, split-K (few tiles, long K), the 8-wave variant (at
# most one workgroup per CU) and the 4-wave one (more tiles than CUs).
MID_SHAPES = [(4, 4, 4), (100, 68, 36), (130, 196, 260), (60, 4, 1028), (64, 64, 64),
              (1024, 1024, 1024), (200, 64, 4100), (2052, 1024, 132), (68, 2000, 516)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("M,N,K", MID_SHAPES)
def test_gemm_mid_kernel(tlib, M, N, K, ta, tb):
    A = u(K, M) if ta else u(M, K)
    B = u(N, K) if tb else u(K, N)
    Am = A.T if ta else A
    Bm = B.T if tb else B
    ref = Am.astype(np.float64) @ Bm.astype(np.float64)
    C = run_gemm(tlib, M, N, K, ta, tb, A, B)
    norm, rel = gemm_err(C, ref, K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)
    # the other kernels agree to the same bar
    check(tlib.tth_gemm_mid(0), "mid off")
    try:
        C2 = run_gemm(tlib, M, N, K, ta, tb, A, B)
    finally:
        check(tlib.tth_gemm_mid(1), "mid on")
    norm2, _ = gemm_err(C, C2, K, 1.0, 1.0)
    assert norm2 <= GEMM_TOL, norm2


# The 8- and 4-wave kernels give each wave a load ring of its own (its 8-k
# slice of every tile, no barrier in the K loop); the variants that share
# each tile between the waves sum the same products in the same order: same
# bits, aligned (16-byte loads) and ragged (4-byte loads) operands, split-K
# and grids of more tiles than CUs (the 4-wave kernel) too.
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (1000, 1003, 997), (200, 64, 4100),
                                   (130, 196, 2600), (515, 1025, 1023), (2052, 1024, 132),
                                   (1100, 2000, 262)])
def test_gemm_mid_private_ring_bits(tlib, M, N, K, ta, tb):
    A = u(K, M) if ta else u(M, K)
    B = u(N, K) if tb else u(K, N)
    print("gemm mid rings", M, N, K, ta, tb, flush=True)
    C = run_gemm(tlib, M, N, K, ta, tb, A, B)
    check(tlib.tth_gemm_mid(2), "mid shared ring")
    try:
        C2 = run_gemm(tlib, M, N, K, ta, tb, A, B)
    finally:
        check(tlib.tth_gemm_mid(1), "mid on")
    assert bits_equal(C, C2)
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    norm, rel = gemm_err(C, ref, K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


# Edges of the 64x64 kernel's rings at sizes where it does not run by itself
# (tth_gemm_mid_force): K tails where most waves' 8-k slices lie past K (K =
# 4, 12, 36), partial edge tiles in M and N, split-K over short K chunks,
# 16-byte loads (aligned) and 4-byte loads (K, M or N ragged), both rings
# against each other (same bits) and against float64.
MID_EDGE_SHAPES = [(4, 4, 4), (64, 64, 64), (100, 68, 36), (60, 4, 1028), (130, 196, 260),
                   (68, 132, 12), (17, 13, 5), (33, 70, 99), (5, 300, 3), (300, 260, 1001)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", MID_EDGE_SHAPES)
def test_gemm_mid_forced_edges(tlib, M, N, K, ta, tb):
    A = u(K, M) if ta else u(M, K)
    B = u(N, K) if tb else u(K, N)
    print("gemm mid forced", M, N, K, ta, tb, flush=True)
    check(tlib.tth_gemm_mid_force(1), "mid force")
    try:
        C = run_gemm(tlib, M, N, K, ta, tb, A, B)
        check(tlib.tth_gemm_mid(2), "mid shared ring")
        C2 = run_gemm(tlib, M, N, K, ta, tb, A, B)
    finally:
        check(tlib.tth_gemm_mid(1), "mid on")
        check(tlib.tth_gemm_mid_force(0), "mid force off")
    assert bits_equal(C, C2)
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    norm, rel = gemm_err(C, ref, K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


# Small GEMMs (2MNK < 2^29, >= 128 tiles of 32x32) run the register kernel
# that splits K over the waves of one workgroup: edges in M / N, K not a
# multiple of 8 or below 8, every layout (k-contiguous operands with aligned
# rows take 16-byte loads; the unaligned K = 5 / 13 cases run the layouts
# whose operands are m/n-contiguous).
SMALL_SHAPES = [(300, 500, 36), (257, 513, 256), (4097, 10, 128), (33, 4100, 5), (512, 512, 512),
                (600, 300, 13), (1000, 40, 1000)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", SMALL_SHAPES)
def test_gemm_small_kernel(tlib, M, N, K, ta, tb):
    A = u(K, M) if ta else u(M, K)
    B = u(N, K) if tb else u(K, N)
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    print("gemm small", M, N, K, ta, tb, flush=True)
    C = run_gemm(tlib, M, N, K, ta, tb, A, B)
    norm, rel = gemm_err(C, ref, K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)
    check(tlib.tth_gemm_small(0), "small off")
    try:
        C2 = run_gemm(tlib, M, N, K, ta, tb, A, B)
    finally:
        check(tlib.tth_gemm_small(1), "small on")
    norm2, _ = gemm_err(C, C2, K, 1.0, 1.0)
    assert norm2 <= GEMM_TOL, norm2


# Large GEMMs with unaligned operands are read in place by the 64x64 kernel's
# 4-byte loads: ragged leading dimensions, K % 4 != 0, odd M / N.
PAD_SHAPES = [(1000, 1003, 997), (1001, 1024, 1000), (1024, 999, 1024), (515, 1025, 1023)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", PAD_SHAPES)
def test_gemm_padded_operands(tlib, M, N, K, ta, tb):
    A = u(K, M) if ta else u(M, K)
    B = u(N, K) if tb else u(K, N)
    Am = A.T if ta else A
    Bm = B.T if tb else B
    ref = Am.astype(np.float64) @ Bm.astype(np.float64)
    C = run_gemm(tlib, M, N, K, ta, tb, A, B)
    norm, rel = gemm_err(C, ref, K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


# The same 4-byte-load path for each of the kernel's three tilings (one
# workgroup per CU; more tiles than CUs; tall 256-row tiles), and for
# operands whose first element is not 16-byte aligned.
DW_SHAPES = [(2000, 1999, 1001, 0), (65537, 63, 255, 0), (1024, 1024, 1024, 1), (768, 1000, 1003, 3)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K,shift", DW_SHAPES)
def test_gemm_unaligned_in_place(tlib, M, N, K, shift, ta, tb):
    A = u(K, M) if ta else u(M, K)
    B = u(N, K) if tb else u(K, N)
    Am = A.T if ta else A
    Bm = B.T if tb else B
    ref = Am.astype(np.float64) @ Bm.astype(np.float64)
    # operands start `shift` floats into their buffers
    pa = np.concatenate([np.zeros(shift, np.float32), A.ravel()])
    pb = np.concatenate([np.zeros(shift, np.float32), B.ravel()])
    dA, dB, dC = DevBuf.from_np(pa), DevBuf.from_np(pb), DevBuf(M * N)
    print(f"gemm in place M={M} N={N} K={K} shift={shift} ta={ta} tb={tb}", flush=True)
    check(tlib.tt_k_gemm(M, N, K, dA.ptr + 4 * shift, A.shape[1], ta, dB.ptr + 4 * shift,
                         B.shape[1], tb, dC.ptr, N), "tt_k_gemm")
    C = dC.to_np((M, N))
    norm, rel = gemm_err(C, ref, K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


def test_gemm_unaligned_nonfinite_isolation(tlib):
    """In-place reads of ragged rows touch no element outside the operand's
    own rows / columns: an Inf at the start of a row of A and a NaN at the
    end of the last row of B reach only their own row / column of C."""
    M, N, K = 1000, 997, 1003
    A, B = u(M, K), u(K, N)
    A[5, 0] = np.inf
    A[6, K - 1] = np.inf
    B[K - 1, N - 1] = np.nan
    C = run_gemm(tlib, M, N, K, 0, 0, A, B)
    bad = ~np.isfinite(C)
    expect = np.zeros_like(bad)
    expect[5, :] = expect[6, :] = True
    expect[:, N - 1] = True
    assert np.array_equal(bad, expect)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    keep = ~expect
    norm, rel = gemm_err(C[keep], ref[keep], K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


# Tall GEMMs with few columns (N <= 64, at least 256 tiles of 256 rows) take
# the 256-row tiles of the 64x64 kernel: edge rows and columns, a K tail,
# all three transposition layouts, whole result against float64.
TALL_SHAPES = [(65536, 64, 256), (65600, 48, 200), (70000, 60, 132)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("M,N,K", TALL_SHAPES)
def test_gemm_tall_rows(tlib, M, N, K, ta, tb):
    A = u(K, M) if ta else u(M, K)
    B = u(N, K) if tb else u(K, N)
    Am = A.T if ta else A
    Bm = B.T if tb else B
    ref = Am.astype(np.float64) @ Bm.astype(np.float64)
    C = run_gemm(tlib, M, N, K, ta, tb, A, B)
    norm, rel = gemm_err(C, ref, K, 1.0, 1.0)
    assert norm <= GEMM_TOL and rel <= GEMM_TOL, (norm, rel)


@pytest.mark.parametrize("rows,cols", [(1, 10), (128, 10), (256, 10), (512, 33), (300, 7)])
def test_softmax_ce_mean_host_labels(tlib, rows, cols):
    """Labels in the launch arguments: bit for bit the device-label kernel,
    out-of-range labels included."""
    x = (rng.standard_normal((rows, cols)) * 4).astype(np.float32)
    y = rng.integers(0, cols, rows).astype(np.int32)
    y[:: 17] = cols + 3
    outs = []
    for host in (False, True):
        dx_, dp, ds, dl = DevBuf.from_np(x), DevBuf(rows * cols), DevBuf(rows * cols), DevBuf(1)
        if host:
            check(tlib.tt_k_softmax_ce_mean_hostlab(dx_.ptr, y.ctypes.data, dp.ptr, dl.ptr, ds.ptr, rows,
                                                    cols, ctypes.c_float(1.0 / rows)), "hostlab")
        else:
            dlab = DevBuf.from_np(y)
            check(tlib.tt_k_softmax_ce_mean(dx_.ptr, dlab.ptr, dp.ptr, dl.ptr, ds.ptr, rows, cols,
                                            ctypes.c_float(1.0 / rows)), "devlab")
        outs.append([dp.to_np((rows, cols)), ds.to_np((rows, cols)), dl.to_np((1,))])
    for a, b in zip(*outs):
        assert bits_equal(a, b)
    assert tlib.tt_k_softmax_ce_mean_hostlab(dx_.ptr, y.ctypes.data, dp.ptr, dl.ptr, ds.ptr, 513, cols,
                                             ctypes.c_float(1.0)) == -1


def test_autograd_softmax_ce_seed_moves_and_recomputes(tlib):
    """ag_softmax_ce backward: the first backward with the default seed hands
    the logits the per-row seed (p - onehot)/rows; a second backward adds the
    recomputed seed (exactly twice the first); a seed of 2 scales it."""
    from tinytorch_amd.torch_py import Node
    rows, cols = 128, 10
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    y = rng.integers(0, cols, rows).astype(np.int32)
    X = Node.leaf(x)
    loss = X.softmax_ce(y)
    p = loss.probs()
    onehot = np.eye(cols, dtype=np.float32)[y]
    seed = (p - onehot) * np.float32(1.0 / rows)
    loss.backward(None)
    g1 = X.grad()
    assert bits_equal(g1, seed)
    assert bits_equal(loss.grad(), np.ones(1, np.float32))
    loss.backward(None)
    assert bits_equal(X.grad(), seed + seed)
    loss.release()
    X.release()
    X2 = Node.leaf(x)
    loss2 = X2.softmax_ce(y)
    loss2.backward(np.array([2.0], np.float32))
    assert bits_equal(X2.grad(), seed * np.float32(2.0))
    loss2.release()
    X2.release()
