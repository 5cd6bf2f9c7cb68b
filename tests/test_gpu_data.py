"""Device-resident datasets: the batch gather + normalise kernel must equal
the oracle's NumPy restatement of the harnesses' normalisation bit for bit,
on files written from the idx / CIFAR-10 binary format definitions."""
import gzip
import os
import struct
import sys

import numpy as np
import pytest

import orc

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
rng = np.random.default_rng(77)


@pytest.fixture(scope="module")
def data(tlib):
    from tinytorch_amd import data as _data
    return _data


@pytest.fixture(scope="module")
def pb(tlib):
    sys.path.insert(0, os.path.join(ROOT, "build"))
    try:
        import tinytorch_pybind
    finally:
        sys.path.pop(0)
    return tinytorch_pybind


def write_idx(path, arr, gz=True):
    raw = struct.pack(">BBBB", 0, 0, 8, arr.ndim) + struct.pack(">" + "I" * arr.ndim, *arr.shape)
    raw += np.ascontiguousarray(arr, np.uint8).tobytes()
    with (gzip.open(path, "wb") if gz else open(path, "wb")) as f:
        f.write(raw)


@pytest.fixture(scope="module")
def mnist_files(tmp_path_factory):
    d = tmp_path_factory.mktemp("mnist")
    img = rng.integers(0, 256, (1000, 28, 28), dtype=np.uint8)
    lab = rng.integers(0, 10, 1000).astype(np.uint8)
    write_idx(str(d / "train-images-idx3-ubyte.gz"), img)
    write_idx(str(d / "train-labels-idx1-ubyte.gz"), lab)
    write_idx(str(d / "plain-images"), img, gz=False)
    return str(d / "train-images-idx3-ubyte.gz"), str(d / "train-labels-idx1-ubyte.gz"), \
        str(d / "plain-images"), img, lab


@pytest.fixture(scope="module")
def cifar_files(tmp_path_factory):
    d = tmp_path_factory.mktemp("cifar")
    paths = []
    for i, n in enumerate((300, 211)):
        im = rng.integers(0, 256, (n, 3, 32, 32), dtype=np.uint8)
        lb = rng.integers(0, 10, n).astype(np.uint8)
        recs = np.concatenate([lb[:, None], im.reshape(n, -1)], axis=1)
        p = str(d / f"data_batch_{i + 1}.bin")
        recs.tofile(p)
        paths.append(p)
    return paths


def test_mnist_batches_bit_exact(data, mnist_files):
    ip, lp, plain, img, lab = mnist_files
    ds = data.Dataset.mnist(ip, lp)
    assert len(ds) == 1000 and ds.shape == (1, 28, 28)
    assert np.array_equal(ds.labels(), lab.astype(np.int32))
    ref_all = orc.normalize_u8(orc.read_idx(ip)[:, None], [0.1307], [0.3081])
    order = rng.permutation(1000)
    for start, bs in ((0, 128), (128, 256), (384, 1), (385, 615)):
        idx = order[start:start + bs]
        node, y = ds.batch(idx, flat=True)
        got = node.value()
        assert got.shape == (len(idx), 784)
        assert np.array_equal(got, ref_all[idx].reshape(len(idx), 784))
        assert np.array_equal(y, lab[idx].astype(np.int32))
        node.release()
    # the plain (not gzip'd) file reads the same
    ds2 = data.Dataset.mnist(plain, lp)
    n2, _ = ds2.batch(np.arange(10))
    assert np.array_equal(n2.value(), ref_all[:10])
    n2.release()
    for d in (ds, ds2):
        d.release()


def test_cifar_batches_bit_exact(data, pb, cifar_files):
    x, y = orc.read_cifar_bin(cifar_files)
    ref_all = orc.normalize_u8(x, data.CIFAR_MEAN, data.CIFAR_STD)
    ds = data.Dataset.cifar10(cifar_files)
    assert len(ds) == 511 and ds.shape == (3, 32, 32)
    idx = rng.permutation(511)[:256]
    node, lab = ds.batch(idx)
    assert np.array_equal(node.value(), ref_all[idx])
    assert np.array_equal(lab, y[idx])
    node.release()
    ds.release()
    # the pybind module's Dataset
    dp = pb.Dataset.cifar10(cifar_files)
    assert len(dp) == 511
    n3, lab3 = dp.batch(idx)
    assert np.array_equal(n3.value(), ref_all[idx]) and np.array_equal(lab3, y[idx])


def test_scalar_path_and_errors(data, mnist_files, tmp_path):
    """sample planes that are not a multiple of 4 take the scalar kernel;
    bad indices, malformed files and mismatched mean/std fail loudly"""
    xs = rng.integers(0, 256, (40, 3, 5, 5), dtype=np.uint8)
    ls = rng.integers(0, 10, 40).astype(np.int32)
    mean, std = (0.5, 0.25, 0.125), (0.3, 0.2, 0.1)
    ds = data.Dataset.from_u8(xs, ls, mean, std)
    idx = np.array([39, 0, 7, 7, 12])
    node, lab = ds.batch(idx)
    assert np.array_equal(node.value(), orc.normalize_u8(xs, mean, std)[idx])
    assert np.array_equal(lab, ls[idx])
    node.release()
    with pytest.raises(ValueError):
        ds.batch(np.array([0, 40]))
    with pytest.raises(ValueError):
        ds.batch(np.array([-1]))
    ds.release()
    ip, lp, _, _, _ = mnist_files
    with pytest.raises(ValueError):
        data.Dataset.mnist(ip, ip)  # labels file with 3 dims
    bad = str(tmp_path / "bad.bin")
    np.zeros(3073 + 5, np.uint8).tofile(bad)  # not a whole number of records
    with pytest.raises(ValueError):
        data.Dataset.cifar10([bad])
    with pytest.raises(ValueError):
        data.Dataset.mnist(ip, lp, mean=(0.1, 0.2), std=(0.3, 0.4))


def test_mlp_step_from_device_batches(data, mnist_files):
    """An MLP step whose input batch comes from the device dataset gives the
    oracle's step on the same (host-normalised) batch."""
    from tinytorch_amd.torch_py import Node
    ip, lp, _, img, lab = mnist_files
    ds = data.Dataset.mnist(ip, lp)
    _, _, Ws = orc.mlp_inputs(B=128)
    idx = rng.permutation(1000)[:128]
    X, y = ds.batch(idx, flat=True)
    xh = orc.normalize_u8(img[idx][:, None], [0.1307], [0.3081]).reshape(128, 784)
    ref = orc.mlp_step(xh, y, *Ws)
    ws = [Node.leaf(w) for w in Ws]
    h = X.padones().matmul(ws[0]).relu().padones().matmul(ws[1]).relu().padones()
    logits = h.matmul(ws[2])
    loss = logits.softmax_ce(y)
    loss.backward()
    for w, k in zip(ws, ("dW1", "dW2", "dW3")):
        r = ref[k]
        assert np.abs(w.grad() - r).max() <= 1e-4 * np.abs(r).max(), k
    for n in [loss, logits, h, X] + ws:
        n.release()
    ds.release()
