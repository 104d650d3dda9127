"""The leaf producer, the both-OOB proximity and the one-hot low-rank
products: the library's kernels run on the CPU by the emulator (tests/emu,
script mode), through the C ABI, against the oracle.  Bars as in the GPU
tests: identical node indices, OOB words, counts and float quotients;
P V within 1e-5 and Q B Q^T within 1e-4 relative Frobenius of double
evaluations.  Sizes are cut to what the emulation runs in seconds."""
import numpy as np
import pytest

import oracle as O
from emu_session import CTX, EmuScript
from test_emu_cpu import pack_words
from test_oracle import random_features, random_forest_arrays, sklearn_forest


def terminal(f, leaf):
    return np.where(np.take_along_axis(f["nodestatus"], np.maximum(leaf, 0), axis=1) == -1, leaf, -1).astype(np.int32)


def leaves_call(s, mode, f, X, nin=None, terminal_only=0, oob=False):
    t, maxnode = f["nodestatus"].shape
    n, mdim = X.shape
    cg, cat = f.get("catgoleft"), f.get("cat")
    maxcat = 1 if cg is None else cg.shape[2]
    leaf = s.out(4 * t * n)
    ld = (n + 31) // 32
    words = s.out(4 * t * ld) if oob else None
    s.call("rfxp_forest_leaves", CTX, mode, s.dev(f["nodestatus"]), s.dev(f["bestvar"]), s.dev(f["xbestsplit"]),
           s.dev(f["treemap"]), None if cg is None else s.dev(cg), None if cat is None else s.dev(cat), t, maxnode,
           maxcat, mdim, s.dev(X), n, None if nin is None else s.dev(nin), terminal_only, leaf, words,
           ld if oob else 0)
    return leaf, words


@pytest.mark.parametrize("n,t,maxnode", [(1, 3, 5), (333, 17, 41), (2000, 24, 257)])
def test_leaves_every_mode(emu_driver, tmp_path, n, t, maxnode):
    rng = np.random.default_rng(n + t)
    cat = [1, 1, 3, 5, 2, 1]
    f = random_forest_arrays(rng, t, maxnode, cat, 5)
    X = random_features(rng, n, cat)
    nin = (rng.random((t, n)) < 0.63).astype(np.int32) * rng.integers(1, 3, (t, n)).astype(np.int32)
    no_cat = dict(f, cat=None, catgoleft=None)
    s = EmuScript(emu_driver)
    pred, _ = leaves_call(s, 0, f, X)
    train, words = leaves_call(s, 1, f, X, nin=nin, oob=True)
    term, _ = leaves_call(s, 1, f, X, nin=nin, terminal_only=1)
    pred_nc, _ = leaves_call(s, 0, no_cat, X)
    assert s.run(tmp_path) == [0] * 4
    assert np.array_equal(pred.array(np.int32, (t, n)), O.forest_leaves(0, f, X))
    want = O.forest_leaves(1, f, X, nin)
    assert np.array_equal(train.array(np.int32, (t, n)), want)
    assert np.array_equal(words.array(np.uint32, (t, (n + 31) // 32)), pack_words((nin == 0).astype(np.uint8)))
    assert np.array_equal(term.array(np.int32, (t, n)), terminal(f, want))
    assert np.array_equal(pred_nc.array(np.int32, (t, n)), O.forest_leaves(0, no_cat, X))


def test_leaves_feed_the_triangle(emu_driver, tmp_path):
    """sklearn CART trees -> training leaves and OOB words -> rfxp_set_forest
    -> rfxp_upper (F32): the oracle's triangle of the same forest."""
    rng = np.random.default_rng(71)
    trees, f, X = sklearn_forest(rng, 12, 700, 5)
    t, maxnode = f["nodestatus"].shape
    n = X.shape[0]
    nin = np.stack([np.bincount(rng.integers(0, n, n), minlength=n) for _ in range(t)]).astype(np.int32)
    s = EmuScript(emu_driver)
    leaf, words = leaves_call(s, 1, f, X, nin=nin, terminal_only=1, oob=True)
    out = s.out(4 * n * (n + 1) // 2)
    s.call("rfxp_set_forest", CTX, leaf, 1, n, words, (n + 31) // 32, n, t, maxnode, None)
    s.call("rfxp_upper", CTX, O.FMT_F32, 1.0, 0.0, 0, n, out)
    assert s.run(tmp_path) == [0, 0, 0]
    want_leaf = terminal(f, O.forest_leaves(1, f, X, nin))
    assert np.array_equal(leaf.array(np.int32, (t, n)), want_leaf)
    want = O.upper_rows(want_leaf, (nin == 0).astype(np.uint8), maxnode, O.FMT_F32)
    assert np.array_equal(out.array(np.float32), want)


@pytest.mark.parametrize("n,t,nleaf", [(1, 5, 2), (63, 32, 4), (65, 70, 3), (300, 40, 9)])
def test_both_oob(emu_driver, tmp_path, n, t, nleaf):
    rng = np.random.default_rng(n + 100 * t)
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    leaf[rng.random((t, n)) < 0.05] = nleaf + 3
    oob = (rng.random((t, n)) < 0.37).astype(np.uint8)
    if n > 1:
        oob[:, 0] = 0
    words = pack_words(oob)
    s = EmuScript(emu_driver)
    lb, wb = s.dev(leaf), s.dev(words)
    lbs = s.dev(np.ascontiguousarray(leaf.T))
    ne = n * (n + 1) // 2
    outs = {}
    for fmt, size in ((O.FMT_F32, 4), (O.FMT_U16, 2)):
        outs[fmt] = s.out(size * ne)
        s.call("rfxp_both_oob", CTX, lb, 1, n, wb, words.shape[1], n, t, nleaf, fmt, 0, n, outs[fmt])
    bands = [(0, n), (n // 3, n // 2 + 1), (n - 1, n)]
    band_outs = []
    for r0, r1 in bands:
        start = lambda r: r * n - r * (r - 1) // 2           # packed index of (r, r); N(N+1)/2 at r = N
        o = s.out(4 * (start(r1) - start(r0)))
        s.call("rfxp_both_oob", CTX, lbs, t, 1, wb, words.shape[1], n, t, nleaf, O.FMT_F32, r0, r1, o)
        band_outs.append(o)
    assert s.run(tmp_path) == [0] * (2 + len(bands))
    assert np.array_equal(outs[O.FMT_F32].array(np.float32), O.both_oob_rows(leaf, oob, nleaf, O.FMT_F32))
    assert np.array_equal(outs[O.FMT_U16].array(np.uint16), O.both_oob_rows(leaf, oob, nleaf, O.FMT_U16))
    for (r0, r1), o in zip(bands, band_outs):
        assert np.array_equal(o.array(np.float32), O.both_oob_rows(leaf, oob, nleaf, O.FMT_F32, r0, r1)), (r0, r1)


def zipf_leaves(rng, n, t, nleaf, s=1.1):
    p = 1.0 / np.arange(1, nleaf + 1) ** s
    p /= p.sum()
    leaf = np.empty((t, n), dtype=np.int32)
    for k in range(t):
        perm = rng.permutation(nleaf).astype(np.int32)
        leaf[k] = perm[rng.choice(nleaf, size=n, p=p)]
    return leaf


def rel_fro(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("n,t,nleaf,r", [(1, 1, 1, 1), (300, 7, 5, 3), (5000, 20, 40, 32), (9000, 9, 3, 64)])
def test_lowrank_pv(emu_driver, tmp_path, n, t, nleaf, r):
    """Skewed leaves: the big ones span several pieces (float atomics)."""
    rng = np.random.default_rng(n + r)
    leaf = zipf_leaves(rng, n, t, nleaf)
    if n > 100:
        leaf[rng.random((t, n)) < 0.03] = -1
    V = rng.standard_normal((n, r)).astype(np.float32)
    s = EmuScript(emu_driver)
    Y = s.out(4 * n * r)
    s.call("rfxp_set_reference", CTX, s.dev(leaf), 1, n, n, t, nleaf)
    s.call("rfxp_lowrank_pv", CTX, s.dev(V), r, Y)
    assert s.run(tmp_path) == [0, 0]
    want = O.lowrank_pv(leaf, nleaf, V.astype(np.float64))
    assert rel_fro(Y.array(np.float32, (n, r)).astype(np.float64), want) < 1e-5


def test_lowrank_subspace(emu_driver, tmp_path):
    rng = np.random.default_rng(4)
    n, t, nleaf, r, iters = 3000, 20, 24, 8, 5
    leaf = zipf_leaves(rng, n, t, nleaf)
    V0 = rng.standard_normal((n, r)).astype(np.float32)
    s = EmuScript(emu_driver)
    Q = s.out(4 * n * r)
    B = s.out(8 * r * r, host=True)
    s.call("rfxp_set_reference", CTX, s.dev(leaf), 1, n, n, t, nleaf)
    s.call("rfxp_lowrank_subspace", CTX, s.dev(V0), r, iters, Q, B)
    assert s.run(tmp_path) == [0, 0]
    Qg = Q.array(np.float32, (n, r)).astype(np.float64)
    Bg = B.array(np.float64, (r, r))

    def orth(X):
        q, R = np.linalg.qr(X)
        return q * np.sign(np.diag(R))

    Qw = orth(V0.astype(np.float64))
    for _ in range(iters):
        Qw = orth(O.lowrank_pv(leaf, nleaf, Qw))
    Bw = Qw.T @ O.lowrank_pv(leaf, nleaf, Qw)
    assert np.abs(Qg.T @ Qg - np.eye(r)).max() < 1e-5
    Vt = rng.standard_normal((n, r))
    assert rel_fro(Qg @ (Bg @ (Qg.T @ Vt)), Qw @ (Bw @ (Qw.T @ Vt))) < 1e-4
