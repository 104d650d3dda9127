"""GPU parity of the leaf-assignment producer (rfxp_forest_leaves) against the
oracle's restatement of the reference's three tree walks, which
tests/test_oracle.py pins to the compiled cpu_testreebag, to sklearn's
apply() and, composed with the proximity, to the compiled cpu_proximity.
Bar: identical node indices and OOB words; end to end, identical triangles."""
import numpy as np
import pytest

import oracle as O
import rfxprox as R
from test_oracle import random_features, random_forest_arrays, sklearn_forest

pytestmark = pytest.mark.gpu


def dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def dev_forest(f):
    return {k: dev(v) for k, v in f.items() if v is not None}


def terminal(f, leaf):
    return np.where(np.take_along_axis(f["nodestatus"], np.maximum(leaf, 0), axis=1) == -1, leaf, -1).astype(np.int32)


@pytest.mark.parametrize("n,t,maxnode", [(1, 3, 5), (333, 17, 41), (5000, 40, 257)])
def test_leaves_match_oracle(gpu_ctx, n, t, maxnode):
    import torch

    rng = np.random.default_rng(n + t)
    cat = [1, 1, 3, 5, 2, 1]
    f = random_forest_arrays(rng, t, maxnode, cat, 5)
    X = random_features(rng, n, cat)
    nin = (rng.random((t, n)) < 0.63).astype(np.int32) * rng.integers(1, 3, (t, n)).astype(np.int32)
    fd, Xd = dev_forest(f), dev(X)
    got = gpu_ctx.forest_leaves(R.LEAVES_PREDICT, fd, Xd).cpu().numpy()
    assert np.array_equal(got, O.forest_leaves(0, f, X))
    leaf, words = gpu_ctx.forest_leaves(R.LEAVES_TRAIN, fd, Xd, nin=dev(nin), oob=True)
    want = O.forest_leaves(1, f, X, nin)
    assert np.array_equal(leaf.cpu().numpy(), want)
    assert np.array_equal(words.cpu().numpy(), R.pack_oob_bits(dev(nin == 0).to(torch.bool)).cpu().numpy())
    term = gpu_ctx.forest_leaves(R.LEAVES_TRAIN, fd, Xd, nin=dev(nin), terminal_only=True).cpu().numpy()
    assert np.array_equal(term, terminal(f, want))
    no_cat = dict(f, cat=None, catgoleft=None)
    got = gpu_ctx.forest_leaves(R.LEAVES_PREDICT, dev_forest(no_cat), Xd).cpu().numpy()
    assert np.array_equal(got, O.forest_leaves(0, no_cat, X))


def test_leaves_feed_the_triangle(gpu_ctx):
    """Trees (sklearn CART) -> training leaves and OOB bits on the device ->
    rfxp_set_forest -> rfxp_upper: the oracle's triangle of the same forest."""
    rng = np.random.default_rng(71)
    trees, f, X = sklearn_forest(rng, 24, 1500, 5)
    t, maxnode = f["nodestatus"].shape
    n = X.shape[0]
    nin = np.stack([np.bincount(rng.integers(0, n, n), minlength=n) for _ in range(t)]).astype(np.int32)
    leaf, words = gpu_ctx.forest_leaves(R.LEAVES_TRAIN, dev_forest(f), dev(X), nin=dev(nin), terminal_only=True,
                                        oob=True)
    gpu_ctx.set_forest(leaf, words, n, t, maxnode)
    import torch

    out = torch.empty(R.upper_nbytes(R.FMT_F32, n) // 4, dtype=torch.float32, device="cuda:0")
    gpu_ctx.upper(R.FMT_F32, out, 0, n)
    torch.cuda.synchronize()
    want_leaf = terminal(f, O.forest_leaves(1, f, X, nin))
    assert np.array_equal(leaf.cpu().numpy(), want_leaf)
    want = O.upper_rows(want_leaf, (nin == 0).astype(np.uint8), maxnode, O.FMT_F32)
    assert np.array_equal(out.cpu().numpy(), want)


def test_leaves_rejects_bad_arguments(gpu_ctx):
    import ctypes

    L = R.load()
    ns = dev(np.full((2, 3), -1, np.int32))
    host = np.zeros(6, np.int32)
    rc = L.rfxp_forest_leaves(gpu_ctx.h, 7, ns.data_ptr(), ns.data_ptr(), ns.data_ptr(), ns.data_ptr(), None, None,
                              2, 3, 1, 1, ns.data_ptr(), 2, None, 0, ns.data_ptr(), None, 0)
    assert rc == 1  # unknown mode
    rc = L.rfxp_forest_leaves(gpu_ctx.h, 0, host.ctypes.data_as(ctypes.c_void_p), ns.data_ptr(), ns.data_ptr(),
                              ns.data_ptr(), None, None, 2, 3, 1, 1, ns.data_ptr(), 2, None, 0, ns.data_ptr(), None, 0)
    assert rc == 1  # host pointer
    rc = L.rfxp_forest_leaves(gpu_ctx.h, 1, ns.data_ptr(), ns.data_ptr(), ns.data_ptr(), ns.data_ptr(), None, None,
                              2, 3, 1, 1, ns.data_ptr(), 2, None, 0, ns.data_ptr(), None, 0)
    assert rc == 1  # training mode without nin
