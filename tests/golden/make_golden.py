"""Writes tests/golden/ref_vectors.npz: input/output vectors of the reference
library compiled from its own C sources (oracle/_ref, built by
`make -C oracle ref`).  The vectors pin the oracle restatement wherever the
reference build is not available (e.g. on the GPU box).

Run from the repo root:  python tests/golden/make_golden.py
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import orc  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_vectors.npz")


def graph_unary_bwd(op, x, seed, *args):
    """value and input-grad of one reference autograd op"""
    g = orc.RefGraph()
    L = orc.ref()
    X = g.leaf(x)
    Y = g.add(getattr(L, op)(X, *args))
    g.backward(Y, seed)
    y = g.value(Y, seed.shape)
    dx = g.grad(X, x.shape)
    g.release()
    return y, dx


def main():
    if not orc.ref_available():
        sys.exit("oracle/_ref not built: run `make -C oracle ref` first")
    rng = np.random.default_rng(20240601)
    V = {}
    u = lambda *s: rng.uniform(-1, 1, s).astype(np.float32)  # noqa: E731

    # GEMM (blocked kernel + tails), ragged and aligned
    for tag, (M, N, K) in {"g1": (37, 45, 29), "g2": (64, 48, 40), "g3": (5, 20, 9)}.items():
        A, B = u(M, K), u(K, N)
        V[f"{tag}_A"], V[f"{tag}_B"], V[f"{tag}_C"] = A, B, orc.ref_sgemm(A, B)

    # matmul backward (dA = g B^T dot form, dB = A^T g axpy form)
    A, B, G = u(9, 7), u(7, 11), u(9, 11)
    g = orc.RefGraph()
    L = orc.ref()
    nA, nB = g.leaf(A), g.leaf(B)
    nC = g.add(L.ag_matmul(nA, nB))
    g.backward(nC, G)
    V.update(mm_A=A, mm_B=B, mm_G=G, mm_dA=g.grad(nA, A.shape), mm_dB=g.grad(nB, B.shape))
    g.release()

    # conv2d forward + backward: stride 1 pad 1 and stride 2 pad 0
    for tag, (sh, ph) in {"c1": (1, 1), "c2": (2, 0)}.items():
        x, w, b = u(2, 3, 7, 7), u(4, 3, 3, 3), u(4)
        Ho = (7 + 2 * ph - 3) // sh + 1
        G = u(2, 4, Ho, Ho)
        g = orc.RefGraph()
        nx, nw, nb = g.leaf(x), g.leaf(w), g.leaf(b)
        ny = g.add(L.ag_conv2d(nx, nw, nb, sh, sh, ph, ph))
        g.backward(ny, G)
        V.update({f"{tag}_x": x, f"{tag}_w": w, f"{tag}_b": b, f"{tag}_G": G,
                  f"{tag}_y": g.value(ny, G.shape), f"{tag}_dx": g.grad(nx, x.shape),
                  f"{tag}_dw": g.grad(nw, w.shape), f"{tag}_db": g.grad(nb, b.shape)})
        g.release()

    # pools: non-overlapping 2/2 with ties and specials, overlapping 3/2
    xp = u(2, 3, 6, 6)
    xp[0, 0, 0:2, 0:2] = 0.5          # 4-way tie -> first (top-left) wins
    xp[0, 1, :2, :2] = -np.inf        # all -inf -> -inf, grad to top-left
    xp[0, 2, :2, :2] = np.nan         # all NaN -> -inf
    xp[1, 0, 0, 0] = np.nan           # NaN never wins
    for tag, (p, s) in {"mp1": (2, 2), "mp2": (3, 2)}.items():
        Ho = (6 - p) // s + 1
        G = u(2, 3, Ho, Ho)
        y, dx = graph_unary_bwd("ag_maxpool2d", xp, G, p, p, s, s)
        V.update({f"{tag}_x": xp, f"{tag}_G": G, f"{tag}_y": y, f"{tag}_dx": dx})
        xa = u(2, 3, 6, 6)
        y, dx = graph_unary_bwd("ag_avgpool2d", xa, G, p, p, s, s)
        V.update({f"a{tag}_x": xa, f"a{tag}_G": G, f"a{tag}_y": y, f"a{tag}_dx": dx})

    # relu / softmax / padones
    xr = u(5, 8)
    xr[0, :3] = [0.0, np.inf, -np.inf]
    G = u(5, 8)
    V["relu_x"], V["relu_G"] = xr, G
    V["relu_y"], V["relu_dx"] = graph_unary_bwd("ag_relu", xr, G)
    xs = u(6, 10) * 5
    xs[1] = -np.inf
    xs[2] += 100.0
    V["sm_x"], V["sm_G"] = xs, u(6, 10)
    V["sm_y"], V["sm_dx"] = graph_unary_bwd("ag_softmax", xs, V["sm_G"])
    xo = u(4, 6)
    G = u(4, 7)
    V["po_x"], V["po_G"] = xo, G
    V["po_y"], V["po_dx"] = graph_unary_bwd("ag_padones", xo, G)

    # whole steps at miniature sizes
    x, y, Ws = orc.mlp_inputs(B=8, dims=(20, 16, 12, 10), seed=77)
    r = orc.ref_mlp_step(x, y, *Ws)
    V.update(mlp_x=x, mlp_y=y, mlp_W1=Ws[0], mlp_W2=Ws[1], mlp_W3=Ws[2],
             **{f"mlp_{k}": v for k, v in r.items()})
    x, y, P = orc.cnn_inputs(B=4, C0=3, H=8, W=8, F1=4, F2=6, classes=10, seed=78)
    r = orc.ref_cnn_step(x, y, **P)
    V.update(cnn_x=x, cnn_y=y, **{f"cnn_{k}": v for k, v in P.items()},
             **{f"cnn_r_{k}": v for k, v in r.items()})

    np.savez_compressed(OUT, **V)
    print(f"wrote {OUT}: {len(V)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
