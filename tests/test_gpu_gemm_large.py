"""GEMMs of the BASELINE configs at full size, whole result against the oracle.

config 1: 1024^3 NN.
config 3: 4096^3 dA = dC*B^T (NT) and dB = A^T*dC (TN) with dC ~ N(0,1); the
          oracle runs its blocked NN sgemm on explicitly transposed copies
          (the reference's own dot/axpy backward loops are naive and serial).
config 5: 8192^3, ragged 1000x1003x997 and tall-skinny 65536x64x4096.
Headline: 4096^3 NN.

Every entry of C is compared (a mis-addressed tile anywhere fails), with the
bars of /root/reference/bench/bench_gemm_opt.py:73-75 as BASELINE.json
states them: max|C - C_ref| / (sqrt(K) max|A| max|B|) <= 1e-4 and
max|C - C_ref| / max|C_ref| <= 1e-4.  The oracle is the AVX2 OpenMP sgemm
restatement (about 1 TFLOP/s on the box's host cores: 8192^3 takes ~1 s).
Operands are uniform[-1, 1] from fixed seeds, as BASELINE.json states.
"""
import os

import numpy as np
import pytest

import orc
from tinytorch_amd.hip import DevBuf, check

pytestmark = pytest.mark.gpu
TOL = 1e-4
THREADS = max(1, min(16, os.cpu_count() or 1))


def gemm(tlib, M, N, K, ta, tb, dA, dB, dC):
    print(f"gemm M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    lda = M if ta else K
    ldb = K if tb else N
    check(tlib.tt_k_gemm(M, N, K, dA.ptr, lda, ta, dB.ptr, ldb, tb, dC.ptr, N), "tt_k_gemm")


def assert_whole(C, ref, K, amax, bmax):
    assert C.shape == ref.shape
    assert np.isfinite(C).all()
    d = float(np.abs(C - ref).max())
    norm = d / (np.sqrt(K) * amax * bmax)
    rel = d / float(np.abs(ref).max())
    assert norm <= TOL and rel <= TOL, (norm, rel)


def test_config1_1024_full_vs_oracle(tlib):
    A = orc.uniform((1024, 1024), -1, 1, 0x5EED + 1)
    B = orc.uniform((1024, 1024), -1, 1, 0x5EED + 2)
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(1024 * 1024)
    gemm(tlib, 1024, 1024, 1024, 0, 0, dA, dB, dC)
    assert_whole(dC.to_np((1024, 1024)), orc.sgemm(A, B, THREADS), 1024, 1.0, 1.0)


def test_config5_ragged_full_vs_oracle(tlib):
    M, N, K = 1000, 1003, 997
    A = orc.uniform((M, K), -1, 1, 51)
    B = orc.uniform((K, N), -1, 1, 52)
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(M * N)
    gemm(tlib, M, N, K, 0, 0, dA, dB, dC)
    assert_whole(dC.to_np((M, N)), orc.sgemm(A, B, THREADS), K, 1.0, 1.0)


@pytest.mark.parametrize("layout", ["nt", "tn"])
def test_config3_backward_4096_full_vs_oracle(tlib, layout):
    n = 4096
    A = orc.uniform((n, n), -1, 1, 31)
    B = orc.uniform((n, n), -1, 1, 32)
    G = orc.normal((n, n), 1.0, 33)
    dG, dC = DevBuf.from_np(G), DevBuf(n * n)
    gmax = float(np.abs(G).max())
    if layout == "nt":   # dA = dC * B^T   (matmul_nt: B stored N x K)
        dB = DevBuf.from_np(B)
        gemm(tlib, n, n, n, 0, 1, dG, dB, dC)
        ref = orc.sgemm(G, np.ascontiguousarray(B.T), THREADS)
    else:                # dB = A^T * dC   (matmul_tn: A stored K x M)
        dA = DevBuf.from_np(A)
        gemm(tlib, n, n, n, 1, 0, dA, dG, dC)
        ref = orc.sgemm(np.ascontiguousarray(A.T), G, THREADS)
    assert_whole(dC.to_np((n, n)), ref, n, 1.0, gmax)


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (8192, 8192, 8192), (65536, 64, 4096)])
def test_config5_large_full_vs_oracle(tlib, M, N, K):
    A = orc.uniform((M, K), -1, 1, 61)
    B = orc.uniform((K, N), -1, 1, 62)
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(M * N)
    gemm(tlib, M, N, K, 0, 0, dA, dB, dC)
    C = dC.to_np((M, N))
    del dC
    assert_whole(C, orc.sgemm(A, B, THREADS), K, 1.0, 1.0)


def test_tile_misaddressing_would_fail():
    """The whole-matrix check catches one wrong 256x256 tile (sanity of the bar)."""
    M = N = K = 512
    A = orc.uniform((M, K), -1, 1, 7)
    B = orc.uniform((K, N), -1, 1, 8)
    ref = orc.sgemm(A, B, THREADS)
    bad = ref.copy()
    bad[256:, 256:] = (A[:256] @ B)[:, 256:]     # rows of the wrong tile of A
    with pytest.raises(AssertionError):
        assert_whole(bad, ref, K, 1.0, 1.0)
