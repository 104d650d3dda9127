"""rfx::ForestProximity (include/rfx_forest.hpp), the object RandomForest's
proximity queries forward to, driven from C++ (tests/compat/forest_driver)
and compared with the oracle's restatements of the same methods:
compute_proximity_from_leaves, get_top_k_similar (indices and float scores
exact), predict_top_k_similar, get_proximity_matrix (exact) and the full-mode
outlier scores (raw measure to 1e-6 relative, then the host median/MAD)."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

FDRIVER = os.path.join(os.path.dirname(__file__), "compat", "forest_driver")


@pytest.mark.parametrize("n,t,k,nleaf,nq", [(700, 37, 9, 23, 40),
                                          (4000, 60, 12, 300, 64)])   # N x N matrix of 64 MB
def test_forest_proximity_object(tmp_path, n, t, k, nleaf, nq):
    assert os.path.exists(FDRIVER), "tests/compat/forest_driver not built (make -C rfx-fuse_amd driver)"
    rng = np.random.default_rng(81 + n)
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int16)
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    oob[:, 3] = 0                                     # never OOB: no results, proximity 0
    pairs = np.array([[0, 1], [5, 5], [3, 9], [10, 600], [699, 0], [-1, 2], [2, 700]], np.int32)
    qleaf = rng.integers(0, nleaf, (nq, t)).astype(np.int16)
    qleaf[0] = leaf[:, 42]
    classes = rng.integers(0, 3, n).astype(np.int32)
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        np.array([n, t, k], np.int32).tofile(f)
        leaf.tofile(f)
        for i in range(n):
            trees = np.flatnonzero(oob[:, i]).astype(np.int32)
            np.array([len(trees)], np.int32).tofile(f)
            trees.tofile(f)
        np.array([len(pairs)], np.int32).tofile(f)
        pairs.tofile(f)
        np.array([nq], np.int32).tofile(f)
        qleaf.tofile(f)
        classes.tofile(f)
    r = subprocess.run(["timeout", "-k", "10", "120", FDRIVER, str(inp), str(outp)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    raw = np.fromfile(outp, np.uint8)
    off = 0

    def take(count, dt):
        nonlocal off
        nb = count * np.dtype(dt).itemsize
        a = raw[off:off + nb].view(dt)
        off += nb
        return a

    L = leaf.astype(np.int32)
    pp = take(len(pairs), np.float32)
    for (a, b), v in zip(pairs, pp):
        assert v == O.pair_proximity(L, oob, nleaf, a, b), (a, b)

    def take_topk():
        m = int(take(1, np.int32)[0])
        rec = take(2 * m, np.int32).reshape(m, 2)
        return rec[:, 0], rec[:, 1].view(np.float32)

    checked = set(range(n)) if n <= 1000 else set(range(0, n, 37)) | {3, 42, n - 1}
    for q in range(n):
        gi, gs = take_topk()
        if q not in checked:
            continue
        wi, wc, ws = O.topk_oob(L, oob, q, k, exclude_self=True)
        assert np.array_equal(gi, wi) and np.array_equal(gs, ws), q
    for q in range(5):
        gi, gs = take_topk()
        wi, wc, ws = O.topk_oob(L, oob, q, k, exclude_self=False)
        assert np.array_equal(gi, wi) and np.array_equal(gs, ws), q
    pi = take(nq * k, np.int32).reshape(nq, k)
    ps = take(nq * k, np.float32).reshape(nq, k)
    wi, wc = O.topk_all(L, qleaf.astype(np.int32), k)
    assert np.array_equal(pi, wi) and np.array_equal(ps, wc.astype(np.float32) / np.float32(t))
    assert pi[0, 0] == 42
    P = take(n * n, np.float32).reshape(n, n)
    tri = O.upper_rows(L, oob, nleaf, O.FMT_F32)
    want = np.zeros((n, n), np.float32)
    want[np.triu_indices(n)] = tri
    want = want + np.triu(want, 1).T
    assert np.array_equal(P, want)
    s0, s1 = take(n, np.float32), take(n, np.float32)
    assert off == raw.size
    rawo = O.outlier_raw(L, nleaf, np.ascontiguousarray(L.T), exclude=np.arange(n, dtype=np.int32),
                         numerator=float(n - 1), isolated=float(n) * 1e10)
    for got, cls in ((s0, None), (s1, classes)):
        want = O.outlier_normalize(rawo, cls)
        assert np.allclose(got, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())
