"""tt_k_gemm_noalloc: the GEMM entry point that allocates no device memory.

Its results are checked bit-for-bit against tt_k_gemm (the same kernels, the
workspace taken from the static scratch array instead of the caching
allocator) on two calls in a row, the second with a smaller input, with
shapes that need workspace (split-K partials, with ragged and with aligned
operands).  A child process whose every library allocation after the
operands fails (TT_FAIL_ALLOC_AFTER) shows that the entry point allocates
nothing: tt_k_gemm fails there, tt_k_gemm_noalloc does not.  A shape whose
workspace exceeds the scratch is refused with TT_E_SCRATCH and C untouched.
"""
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

from tinytorch_amd.hip import DevBuf, check, sync

pytestmark = pytest.mark.gpu
TT_E_SCRATCH = -4
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# (M, N, K): ragged 256x251x8191 takes 16 split-K partials read in place
# (4 MiB); 128x128x8192 takes 64 (4 MiB) of a smaller output
CALLS = [(256, 251, 8191), (128, 128, 8192)]


def operands(M, N, K, seed):
    r = np.random.default_rng(seed)
    return (r.uniform(-1, 1, (M, K)).astype(np.float32),
            r.uniform(-1, 1, (K, N)).astype(np.float32))


def run(tlib, fn, M, N, K, A, B):
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(M * N)
    dC.fill(np.nan)
    print(f"{fn} M={M} N={N} K={K}", flush=True)
    check(getattr(tlib, fn)(M, N, K, dA.ptr, K, 0, dB.ptr, N, 0, dC.ptr, N), fn)
    return dC.to_np((M, N))


def test_noalloc_matches_gemm_two_calls(tlib):
    for i, (M, N, K) in enumerate(CALLS):
        A, B = operands(M, N, K, 100 + i)
        used = tlib.tth_bytes_in_use()
        got = run(tlib, "tt_k_gemm_noalloc", M, N, K, A, B)
        want = run(tlib, "tt_k_gemm", M, N, K, A, B)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (M, N, K)
        assert np.isfinite(got).all()
        ref = A.astype(np.float64) @ B.astype(np.float64)
        assert np.abs(got - ref).max() / np.sqrt(K) <= 1e-4
        assert tlib.tth_bytes_in_use() == used


def test_noalloc_refuses_oversized_workspace(tlib):
    M = N = K = 1024
    A, B = operands(M, N, K, 7)
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(M * N)
    dC.fill(3.0)
    sync()
    # 16 forced splits of a 1024^2 output need 64 MiB of partials: refused
    assert tlib.tth_gemm_config(-1, 64) == 0
    try:
        print("noalloc oversized", flush=True)
        rc = tlib.tt_k_gemm_noalloc(M, N, K, dA.ptr, K, 0, dB.ptr, N, 0, dC.ptr, N)
    finally:
        tlib.tth_gemm_config(-1, -1)
    assert rc == TT_E_SCRATCH
    assert tlib.tth_last_error() == TT_E_SCRATCH
    assert np.all(dC.to_np() == 3.0)


CHILD = textwrap.dedent("""
    import sys, numpy as np
    sys.path.insert(0, {root!r})
    import tinytorch_amd
    from tinytorch_amd.hip import DevBuf
    tinytorch_amd.require_gpu()
    L = tinytorch_amd.lib()
    M, N, K = {shape}
    r = np.random.default_rng(5)
    A = r.uniform(-1, 1, (M, K)).astype(np.float32)
    B = r.uniform(-1, 1, (K, N)).astype(np.float32)
    # the three operand buffers are the only allocations the environment allows
    dA, dB, dC = DevBuf.from_np(A), DevBuf.from_np(B), DevBuf(M * N)
    rc_gemm = L.tt_k_gemm(M, N, K, dA.ptr, K, 0, dB.ptr, N, 0, dC.ptr, N)
    rc = L.tt_k_gemm_noalloc(M, N, K, dA.ptr, K, 0, dB.ptr, N, 0, dC.ptr, N)
    C = dC.to_np((M, N))
    np.save({out!r}, C)
    print("rc", rc_gemm, rc, flush=True)
""")


@pytest.mark.parametrize("shape", CALLS)
def test_noalloc_allocates_nothing(tlib, tmp_path, shape):
    M, N, K = shape
    out = str(tmp_path / "c.npy")
    env = dict(os.environ, TT_FAIL_ALLOC_AFTER="3")
    print("child noalloc", shape, flush=True)
    p = subprocess.run([sys.executable, "-c", CHILD.format(root=ROOT, shape=shape, out=out)],
                       env=env, capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    rc_gemm, rc = (int(v) for v in p.stdout.split()[-2:])
    assert rc_gemm == -2      # the allocating entry point needs workspace and cannot get it
    assert rc == 0
    r = np.random.default_rng(5)
    A = r.uniform(-1, 1, (M, K)).astype(np.float32)
    B = r.uniform(-1, 1, (K, N)).astype(np.float32)
    want = run(tlib, "tt_k_gemm", M, N, K, A, B)
    got = np.load(out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
