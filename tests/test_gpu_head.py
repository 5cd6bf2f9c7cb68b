"""The one-launch classifier backward (head.hip) against the oracle and the
unfused path.

tt_k_head_bwd: dW and dA bit-identical to the reference's
matmul_tn / matmul_nt loops (oracle restatement, pinned against the
reference build on the CPU), the padones / reshape / relu copies exact.
Autograd: the CNN and MLP steps with the fusion on and off against the
oracle, within the steps' tolerance.
"""

import numpy as np
import pytest

import orc
from tinytorch_amd.hip import DevBuf, check

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(77)


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(128, 4097, 10), (256, 257, 10), (5, 70, 32), (3, 2, 1)])
@pytest.mark.parametrize("mode", ["plain", "copy", "relu"])
def test_head_bwd_bitexact(tlib, M, K, N, mode):
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    W = rng.standard_normal((K, N)).astype(np.float32)
    G = (rng.standard_normal((M, N)) / M).astype(np.float32)
    R = np.maximum(rng.standard_normal((M, K - 1)).astype(np.float32), 0.0)
    R[0, : min(3, K - 1)] = [0.0, -0.0, 1e-38][: min(3, K - 1)]
    dA_, dW_, dG, dR = DevBuf.from_np(A), DevBuf.from_np(W), DevBuf.from_np(G), DevBuf.from_np(R)
    gw, ga, d1, d2 = DevBuf(K * N), DevBuf(M * K), DevBuf(M * (K - 1)), DevBuf(M * (K - 1))
    print("head_bwd", M, K, N, mode, flush=True)
    check(tlib.tt_k_head_bwd(dA_.ptr, M, K, dW_.ptr, N, dG.ptr, gw.ptr, ga.ptr,
                             d1.ptr if mode != "plain" else None,
                             d2.ptr if mode != "plain" else None,
                             dR.ptr if mode == "relu" else None), "tt_k_head_bwd")
    assert bits_equal(gw.to_np((K, N)), orc.matmul_tn(A, G))
    dA = orc.matmul_nt(G, W)
    assert bits_equal(ga.to_np((M, K)), dA)
    if mode != "plain":
        assert bits_equal(d1.to_np((M, K - 1)), dA[:, :-1])
        want2 = orc.relu_bwd(R, dA[:, :-1]) if mode == "relu" else dA[:, :-1]
        assert bits_equal(d2.to_np((M, K - 1)), want2)


def _cnn(Node, x, y, P, B):
    X = Node.leaf(x, False)
    ws = {k: Node.leaf(v) for k, v in P.items()}
    h = X.conv2d(ws["w1"], ws["b1"], stride=1, pad=1).relu().maxpool2d(2, 2)
    h = h.conv2d(ws["w2"], ws["b2"], stride=1, pad=1).relu().maxpool2d(2, 2)
    logits = h.reshape((B, P["wfc"].shape[0] - 1)).padones().matmul(ws["wfc"])
    loss = logits.softmax_ce(y)
    loss.backward(None)
    out = {k: ws[k].grad() for k in ws}
    out["loss"] = float(loss.value()[0])
    out["logits"] = logits.value()
    for nd in [loss, logits, X] + list(ws.values()):
        nd.release()
    return out


def _mlp(Node, x, y, Ws):
    X = Node.leaf(x, False)
    W = [Node.leaf(w) for w in Ws]
    h = X.padones().matmul(W[0]).relu().padones().matmul(W[1]).relu()
    logits = h.padones().matmul(W[2])
    loss = logits.softmax_ce(y)
    loss.backward(None)
    out = {f"dW{i + 1}": W[i].grad() for i in range(3)}
    out["loss"] = float(loss.value()[0])
    for nd in [loss, logits, h, X] + W:
        nd.release()
    return out


def test_head_fusion_in_steps_on_off(tlib):
    """The CNN (config 4) and MLP (config 2) steps with every fusion on (the
    one-launch classifier backward) and off (separate GEMMs and padones
    backward) against the oracle, gradients within 1e-4 of their scale."""
    from tinytorch_amd.torch_py import Node
    x, y, P = orc.cnn_inputs()
    ref = orc.cnn_step(x, y, **P)
    xm, ym, Ws = orc.mlp_inputs()
    refm = orc.mlp_step(xm, ym, *Ws)
    prev = tlib.tth_conv_relu_fuse(-1)
    try:
        for on in (1, 0):
            tlib.tth_conv_relu_fuse(on)
            print("steps with fusion", on, flush=True)
            got = _cnn(Node, x, y, P, 128)
            for k, r in (("w1", "dw1"), ("b1", "db1"), ("w2", "dw2"), ("b2", "db2"),
                         ("wfc", "dwfc")):
                err = np.abs(got[k] - ref[r]).max() / max(np.abs(ref[r]).max(), 1e-30)
                assert err <= 1e-4, (on, k, err)
            assert abs(got["loss"] - ref["loss"]) <= 1e-5 * max(1.0, ref["loss"])
            gm = _mlp(Node, xm, ym, Ws)
            for k in ("dW1", "dW2", "dW3"):
                err = np.abs(gm[k] - refm[k]).max() / max(np.abs(refm[k]).max(), 1e-30)
                assert err <= 1e-4, (on, k, err)
            assert abs(gm["loss"] - refm["loss"]) <= 1e-5 * max(1.0, refm["loss"])
    finally:
        tlib.tth_conv_relu_fuse(prev)


@pytest.mark.parametrize("M,F,H2,W2", [(128, 64, 8, 8), (5, 3, 4, 6), (33, 16, 2, 2)])
def test_head_bwd_pool_bitexact(tlib, M, F, H2, W2):
    """tt_k_head_bwd_pool: the classifier backward also writing the pool +
    relu backward of its reshape's gradient from the pool windows' codes --
    dW, dA, d1, d2 bit for bit tt_k_head_bwd's, dc bit for bit
    tt_k_maxpool2x2_code_relu_bwd of d2 (codes with ties, zero masks and
    every argmax)."""
    K, N = F * H2 * W2 + 1, 10
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    W = rng.standard_normal((K, N)).astype(np.float32)
    G = (rng.standard_normal((M, N)) / M).astype(np.float32)
    codes = rng.integers(0, 64, (M, F, H2, W2)).astype(np.uint8)
    dA_, dW_, dG = DevBuf.from_np(A), DevBuf.from_np(W), DevBuf.from_np(G)
    dcodes = DevBuf.from_np(codes)
    outs = []
    for pooled in (True, False):
        dw, da = DevBuf(K * N), DevBuf(M * K)
        d1, d2 = DevBuf(M * (K - 1)), DevBuf(M * (K - 1))
        dc = DevBuf(M * F * 4 * H2 * W2)
        print("head_bwd_pool", M, F, H2, W2, pooled, flush=True)
        if pooled:
            check(tlib.tt_k_head_bwd_pool(dA_.ptr, M, K, dW_.ptr, N, dG.ptr, dw.ptr, da.ptr, d1.ptr,
                                          d2.ptr, dcodes.ptr, dc.ptr, F, H2, W2), "head pool")
        else:
            check(tlib.tt_k_head_bwd(dA_.ptr, M, K, dW_.ptr, N, dG.ptr, dw.ptr, da.ptr, d1.ptr,
                                     d2.ptr, None), "head")
            check(tlib.tt_k_maxpool2x2_code_relu_bwd(dcodes.ptr, d2.ptr, dc.ptr, M, F, 2 * H2,
                                                     2 * W2, H2, W2), "code bwd")
        outs.append([b.to_np() for b in (dw, da, d1, d2, dc)])
    for a, b in zip(*outs):
        assert bits_equal(a, b)
