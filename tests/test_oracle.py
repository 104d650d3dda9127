"""Pins the CPU oracle (oracle/rfx_oracle.c) before it is trusted as the
checker of the HIP path:
  * against golden fixtures written by the reference's own CPU code
    (tests/golden/make_golden.py, oracle/_ref),
  * against the compiled reference directly when oracle/_ref is built here,
  * against brute force and closed forms for what the reference leaves open
    (quantizers, top-K ordering, low rank)."""
import hashlib
import ctypes
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def replay(nodestatus, nodextr, nin, casewise):
    t, n = nodextr.shape
    prox = np.zeros((n, n), order="F")
    for k in range(t):
        O.cpu_proximity(nodestatus[k].astype(np.int32), nodextr[k].astype(np.int32),
                        nin[k].astype(np.int32), nodestatus.shape[1], prox, casewise)
    return prox


# ---- reference fixtures -------------------------------------------------------

@pytest.mark.parametrize("cw", [0, 1])
def test_cpu_proximity_and_finishprox_match_reference_fixture(cw):
    g = np.load(os.path.join(GOLD, "cpu_prox_small.npz"))
    prox = replay(g["nodestatus"], g["nodextr"], g["nin"], cw)
    assert np.array_equal(prox, g[f"prox_cw{cw}"])
    sym = O.finishprox(g["nout"], prox)
    assert np.array_equal(sym, g[f"proxsym_cw{cw}"])


def test_rfgap_matches_reference_fixture():
    g = np.load(os.path.join(GOLD, "rfgap_small.npz"))
    got = O.rfgap(g["nin"].astype(np.int32), g["nodextr"].astype(np.int32))
    assert np.array_equal(got, g["prox"])


def test_c1_forest_triangle_matches_reference_digests():
    """The first benchmark configuration (N=2000, T=100 CART forest): the oracle's packed
    counts, (float)P and uint8 codes hash to the reference's."""
    g = np.load(os.path.join(GOLD, "c1_forest.npz"))
    lab = g["label"].astype(np.int32)
    oob = (g["nin"] == 0).astype(np.uint8)
    nleaf = int(g["nleaf"])
    U = O.upper_counts_scatter(lab, oob, nleaf)
    assert sha(U) == str(g["sha_u16"])
    assert np.array_equal(U[g["samp_idx"]], g["samp_u"])
    p32 = O.upper_rows(lab, oob, nleaf, O.FMT_F32)
    assert sha(p32) == str(g["sha_p32"])
    u8 = O.upper_rows(lab, oob, nleaf, O.FMT_U8, scale=np.float32(1) / np.float32(255))
    assert sha(u8) == str(g["sha_u8"])
    assert int((U == 0).sum()) - lab.shape[1] == int(g["zero_pairs"])


def test_terminal_leaf_adapter_matches_fixture_labels():
    g = np.load(os.path.join(GOLD, "c1_forest.npz"))
    ns, node, nn = g["nodestatus"].astype(np.int32), g["node"].astype(np.int32), g["nnodes"]
    for k in range(0, node.shape[0], 17):
        lab = O.terminal_leaf(ns[k, :nn[k]], node[k])
        assert np.array_equal(lab, g["label"][k].astype(np.int32))


def compiled_reference():
    """The compiled reference (oracle/_ref), loaded only by the tests that
    use it, so that collecting this module maps no library; skips when it
    was not built (it is built in the build container only)."""
    if not O.ref_available():
        pytest.skip("compiled reference (oracle/_ref) not built here")
    return O.ref()


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_oracle_equals_compiled_reference_random_trees(seed):
    R = compiled_reference()
    rng = np.random.default_rng(seed)
    n, t, nnode = 211, 25, 19
    for cw in (0, 1):
        R.ref_set_config(cw, 0, 2)
        pr = np.zeros((n, n), order="F")
        po = np.zeros((n, n), order="F")
        nout = np.zeros(n, np.int32)
        for _ in range(t):
            ns = np.where(rng.random(nnode) < 0.75, -1, rng.integers(1, 3, nnode)).astype(np.int32)
            nx = rng.integers(-2, nnode + 2, n).astype(np.int32)
            nin = np.bincount(rng.integers(0, n, n), minlength=n).astype(np.int32)
            nout += nin == 0
            R.ref_cpu_proximity(ns, nx, nin, n, nnode, pr.reshape(-1, order="F"))
            O.cpu_proximity(ns, nx, nin, nnode, po, cw)
        assert np.array_equal(pr, po)
        ps = np.zeros((n, n), order="F")
        R.ref_cpu_finishprox(n, nout, pr.reshape(-1, order="F"), ps.reshape(-1, order="F"))
        assert np.array_equal(ps, O.finishprox(nout, po))


def test_triangle_formats_equal_reference_finishprox():
    """Every triangle format derives from the reference's (float)P: the float
    formats equal it, the integer codes equal numpy's independent
    evaluation of the quantizer formula on it."""
    R = compiled_reference()
    rng = np.random.default_rng(7)
    n, t, nleaf = 173, 60, 6
    leaf = rng.integers(-1, nleaf + 1, (t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.4).astype(np.uint8)
    oob[:, 5] = 0  # sample 5 never OOB (nout = 0 is left raw)
    R.ref_set_config(0, 0, 2)
    pr = np.zeros((n, n), order="F")
    for k in range(t):
        ns = -np.ones(nleaf, np.int32)
        R.ref_cpu_proximity(ns, leaf[k], (1 - oob[k]).astype(np.int32), n, nleaf, pr.reshape(-1, order="F"))
    nout = O.nout(oob)
    ps = np.zeros((n, n), order="F")
    R.ref_cpu_finishprox(n, nout, pr.reshape(-1, order="F"), ps.reshape(-1, order="F"))
    iu = np.triu_indices(n)
    P32 = ps[iu].astype(np.float32)
    assert np.array_equal(O.upper_rows(leaf, oob, nleaf, O.FMT_F32), P32)
    assert np.array_equal(O.upper_rows(leaf, oob, nleaf, O.FMT_F16), P32.astype(np.float16).view(np.uint16))
    for scale, zp in ((np.float32(1 / 255.0), np.float32(0)), (np.float32(0.003), np.float32(2.5))):
        want = np.clip(P32 / scale + zp, np.float32(0), np.float32(255)).astype(np.uint8)
        assert np.array_equal(O.upper_rows(leaf, oob, nleaf, O.FMT_U8, scale=scale, zp=zp), want)
        want8 = np.clip(P32 / scale + zp, np.float32(-128), np.float32(127)).astype(np.int8)
        assert np.array_equal(O.upper_rows(leaf, oob, nleaf, O.FMT_I8, scale=scale, zp=zp), want8)


# ---- brute force and invariants ----------------------------------------------

def brute_counts(leaf, oob, nleaf):
    t, n = leaf.shape
    valid = (leaf >= 0) & (leaf < nleaf)
    U = np.zeros((n, n), dtype=np.int64)
    for k in range(t):
        same = (leaf[k][:, None] == leaf[k][None, :]) & valid[k][:, None] & valid[k][None, :]
        xor = oob[k][:, None] != oob[k][None, :]
        U += same & xor
    return U[np.triu_indices(n)]


@pytest.mark.parametrize("n,t,nleaf,pinv", [(1, 3, 2, 0.0), (7, 9, 2, 0.2), (64, 30, 5, 0.1),
                                            (130, 17, 1, 0.0)])
def test_counts_equal_brute_force(n, t, nleaf, pinv):
    rng = np.random.default_rng(n + t)
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    leaf[rng.random((t, n)) < pinv] = -1
    oob = (rng.random((t, n)) < 0.37).astype(np.uint8)
    want = brute_counts(leaf, oob, nleaf)
    assert np.array_equal(O.upper_counts_scatter(leaf, oob, nleaf), want)
    assert np.array_equal(O.upper_rows(leaf, oob, nleaf, O.FMT_U16), want)


def test_count_invariants():
    rng = np.random.default_rng(3)
    n, t, nleaf = 300, 80, 7
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.37).astype(np.uint8)
    U = O.upper_rows(leaf, oob, nleaf, O.FMT_U16).astype(np.int64)
    iu = np.triu_indices(n)
    assert (U[iu[0] == iu[1]] == 0).all()
    assert U.max() <= t
    # row sums of the full symmetric matrix: sum_j U_ij = sum_t |opposite bucket of i|
    full = np.zeros((n, n), np.int64)
    full[iu] = U
    full = full + full.T
    want = np.zeros(n, np.int64)
    for k in range(t):
        for i in range(n):
            want[i] += np.sum((leaf[k] == leaf[k][i]) & (oob[k] != oob[k][i]))
    assert np.array_equal(full.sum(axis=1), want)


def test_row_ranges_tile_the_triangle():
    rng = np.random.default_rng(4)
    n, t, nleaf = 97, 20, 4
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.37).astype(np.uint8)
    full = O.upper_rows(leaf, oob, nleaf, O.FMT_F32)
    parts = [O.upper_rows(leaf, oob, nleaf, O.FMT_F32, r0=a, r1=b)
             for a, b in ((0, 10), (10, 11), (11, 60), (60, 97))]
    assert np.array_equal(np.concatenate(parts), full)


def test_p_special_cases():
    # equal nout: 0.5 * (a + a) == a exactly, so P = (U/2) * (1/n)
    for u in (1, 2, 7, 500):
        for nn in (1, 3, 184, 499):
            assert O.p_value(u, nn, nn) == (u / 2.0) * (1.0 / nn)
    # nout == 0 rows are not scaled (src/rf_finishprox.cpp:48)
    assert O.p_value(4, 0, 0) == 2.0
    assert O.p_value(0, 5, 9) == 0.0


# ---- quantizers ---------------------------------------------------------------

def test_f16_conversion_matches_numpy_round_to_nearest_even():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 6, 20000),
        np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 70000.0, 5.96e-8, 2.98e-8, 1e-9, np.inf, -np.inf],
                 dtype=np.float32),
        # exact ties between two halves
        (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0 ** -11) + np.float32(2.0 ** -12)),
    ]).astype(np.float32)
    got = np.array([O.f32_to_f16(v) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, vals.astype(np.float16).view(np.uint16))


def np_roundf(x):
    x = np.asarray(x, dtype=np.float64)
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def test_integer_quantizers_match_independent_numpy_evaluation():
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.random(5000), rng.random(2000) * 3, np.linspace(0, 1, 1021),
                        -rng.random(500)]).astype(np.float32)
    for scale, zp in ((np.float32(1) / np.float32(255), np.float32(0)),
                      (np.float32(1) / np.float32(127), np.float32(0)),
                      (np.float32(0.0037), np.float32(-3.25))):
        r = v / scale + zp
        want_u8 = np.clip(r, np.float32(0), np.float32(255)).astype(np.uint8)
        want_i8 = np.clip(r, np.float32(-128), np.float32(127)).astype(np.int8)
        assert np.array_equal(np.array([O.q_u8(x, scale, zp) for x in v], np.uint8), want_u8)
        assert np.array_equal(np.array([O.q_i8(x, scale, zp) for x in v], np.int8), want_i8)
    x7 = (v * np.float32(7.0)).astype(np.float32)
    want_nf4 = np.where(v >= 0, np.minimum(7, np_roundf(x7)),
                        np.maximum(8, np_roundf((np.float32(8.0) - x7).astype(np.float32))))
    assert np.array_equal(np.array([O.q_nf4(x) for x in v]), want_nf4.astype(np.uint8))
    # round-half-away-from-zero at the nibble boundaries
    assert O.q_nf4(np.float32(0.5) / np.float32(7.0)) in (0, 1)
    assert O.q_nf4(1.0) == 7 and O.q_nf4(0.0) == 0 and O.q_nf4(-1.0) == 15


def test_u8_scale_rule_matches_reference_minmax_formula():
    s, z = O.u8_scale_from_minmax(0.0, 1.0)
    assert s == np.float32(1) / np.float32(255) and z == 0.0
    s, z = O.u8_scale_from_minmax(0.25, 0.75)
    assert s == (np.float32(0.75) - np.float32(0.25)) / np.float32(255)
    assert z == np.float32(-np.float32(0.25) / np.float32(s))


# ---- top-K ----------------------------------------------------------------------

def brute_topk(ref_leaf, qleaf, K, exclude=None, nleaf=2**31 - 1):
    t, n = ref_leaf.shape
    out_i, out_c = [], []
    for q in range(qleaf.shape[0]):
        ok = (qleaf[q] >= 0) & (qleaf[q] < nleaf)
        cnt = ((ref_leaf == qleaf[q][:, None]) & ok[:, None]).sum(axis=0)
        order = np.lexsort((np.arange(n), -cnt))
        if exclude is not None:
            order = order[order != exclude[q]]
        out_i.append(order[:K])
        out_c.append(cnt[order[:K]])
    return np.array(out_i), np.array(out_c)


def test_topk_all_trees_matches_brute_force_with_ties():
    rng = np.random.default_rng(2)
    n, t, q, nleaf, K = 400, 30, 25, 3, 20   # few leaves: many ties
    ref = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    ql = rng.integers(0, nleaf, (q, t)).astype(np.int32)
    idx, cnt = O.topk_all(ref, ql, K)
    bi, bc = brute_topk(ref, ql, K)
    assert np.array_equal(idx, bi) and np.array_equal(cnt, bc)
    ex = rng.integers(0, n, q).astype(np.int32)
    idx, cnt = O.topk_all(ref, ql, K, exclude=ex)
    bi, bc = brute_topk(ref, ql, K, exclude=ex)
    assert np.array_equal(idx, bi) and np.array_equal(cnt, bc)


def test_topk_invalid_labels_match_nothing():
    """Labels outside [0, nleaf) on both sides: equal invalid labels (-1 and
    -1, 5 and 5 with nleaf 4) are not matches, for new and OOB queries."""
    rng = np.random.default_rng(3)
    n, t, q, nleaf, K = 300, 25, 12, 4, 15
    ref = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    ref[rng.random((t, n)) < 0.2] = -1
    ref[rng.random((t, n)) < 0.1] = 5
    ql = np.ascontiguousarray(ref[:, :q].T)            # the same invalid labels in the queries
    idx, cnt = O.topk_all(ref, ql, K, nleaf=nleaf)
    bi, bc = brute_topk(ref, ql, K, nleaf=nleaf)
    assert np.array_equal(idx, bi) and np.array_equal(cnt, bc)
    idx, cnt = O.topk_all(ref, ql, K)                    # without nleaf, 5 is a valid label
    bi, bc = brute_topk(ref, ql, K)
    assert np.array_equal(idx, bi) and np.array_equal(cnt, bc)
    assert not np.array_equal(bc, brute_topk(ref, ql, K, nleaf=nleaf)[1])
    oob = (rng.random((t, n)) < 0.4).astype(np.uint8)
    for qq in (0, 5):
        idx, cnt, sc = O.topk_oob(ref, oob, qq, K, nleaf=nleaf)
        trees = np.nonzero(oob[:, qq])[0]
        lab = ref[trees, qq]
        c = ((ref[trees] == lab[:, None]) & ((lab >= 0) & (lab < nleaf))[:, None]).sum(axis=0)
        c[qq] = 0
        order = np.lexsort((np.arange(n), -c))
        order = order[c[order] > 0][:K]
        assert np.array_equal(idx, order) and np.array_equal(cnt, c[order])
        assert np.array_equal(sc, c[order].astype(np.float32) * (np.float32(1) / np.float32(len(trees))))


def test_topk_oob_semantics():
    rng = np.random.default_rng(5)
    n, t, nleaf, K = 150, 40, 4, 10
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.37).astype(np.uint8)
    for q in (0, 17, 149):
        idx, cnt, sc = O.topk_oob(leaf, oob, q, K)
        trees = np.nonzero(oob[:, q])[0]
        c = (leaf[trees] == leaf[trees, q][:, None]).sum(axis=0)
        c[q] = 0
        order = np.lexsort((np.arange(n), -c))
        order = order[c[order] > 0][:K]
        assert np.array_equal(idx, order) and np.array_equal(cnt, c[order])
        assert np.array_equal(sc, c[order].astype(np.float32) * (np.float32(1) / np.float32(len(trees))))


# ---- low rank -------------------------------------------------------------------

def test_lowrank_pv_equals_dense_one_hot_product():
    rng = np.random.default_rng(6)
    n, t, nleaf, r = 300, 20, 9, 5
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    leaf[0, :4] = -1
    V = rng.standard_normal((n, r))
    A = np.zeros((n, t * nleaf))
    for k in range(t):
        ok = leaf[k] >= 0
        A[np.nonzero(ok)[0], k * nleaf + leaf[k][ok]] = 1.0
    want = (A @ (A.T @ V)) / t
    got = O.lowrank_pv(leaf, nleaf, V)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


# ---- per-tree triangle formats (cuda/rf_proximity_upper_triangle.cu) -----------
# The reference's per-tree kernels are CUDA and cannot run here; their
# restatement is pinned to the reference's CPU accumulation (itself pinned to
# the golden fixture above): each OOB x in-bag pair of a tree is the term that
# rf::cpu_proximity adds, placed once at (min, max) of the pair.

def tri_dense(vals, n):
    D = np.zeros((n, n))
    D[np.triu_indices(n)] = vals
    return D


def fixture_trees():
    g = np.load(os.path.join(GOLD, "cpu_prox_small.npz"))
    return (g["nodestatus"].astype(np.int32), g["nodextr"].astype(np.int32), g["nin"].astype(np.int32), g)


def test_tree_upper_f16_trees_sum_to_reference_fixture():
    ns, nx, nin, g = fixture_trees()
    t, n = nx.shape
    acc = np.zeros((n, n))
    for k in range(t):
        tri = O.tree_upper(O.FMT_F16, ns[k], nx[k], nin[k])
        acc += tri_dense(tri.view(np.float16).astype(np.float64), n)
    P = g["prox_cw0"]
    assert acc.sum() > 0
    assert np.array_equal(acc, np.triu(P + P.T))


def casewise_tree_terms(ns, nx, nin):
    """rf::cpu_proximity of one tree (casewise weights), symmetrised and
    folded to the upper triangle: the weight of each OOB x in-bag pair."""
    n = len(nx)
    P = np.zeros((n, n), order="F")
    O.cpu_proximity(ns, nx, nin, len(ns), P, True)
    return np.triu(P + P.T)


def test_tree_upper_casewise_f16_and_nf4_follow_cpu_pairs():
    ns, nx, nin, _ = fixture_trees()
    n = nx.shape[1]
    for k in range(0, nx.shape[0], 4):
        W = casewise_tree_terms(ns[k], nx[k], nin[k])
        f16 = tri_dense(O.tree_upper(O.FMT_F16, ns[k], nx[k], nin[k], casewise=True).view(np.float16)
                        .astype(np.float64), n)
        assert np.array_equal(f16 > 0, W > 0)
        assert np.abs(f16 - W).max() <= 2.0 ** -11 * W.max()
        nf = O.tree_upper(O.FMT_NF4, ns[k], nx[k], nin[k], casewise=True)
        ne = n * (n + 1) // 2
        nib = np.stack([nf & 15, nf >> 4], axis=1).ravel()[:ne]
        w32 = W[np.triu_indices(n)].astype(np.float32)
        x = (w32 * np.float32(7)).astype(np.float64)
        assert np.array_equal(nib, np.minimum(7, np.floor(x + 0.5)).astype(np.uint8))


def i8_pair_brute(ns, nx, nin, scale, zp, n_real=0):
    """The INT8 per-tree kernel summed pair by pair: entry (i, j), i <= j in
    one terminal node, gets q(nin[j]/size) as (n=i, kk=j) when j is in-bag
    and q(nin[i]/size) as (n=j, kk=i) when i is in-bag and i != j."""
    n = len(nx)
    m = n_real if 0 < n_real < n else n
    out = np.zeros(m * (m + 1) // 2, np.int64)
    term = lambda k: 0 <= k < len(ns) and ns[k] == -1  # noqa: E731
    size = {}
    for s in range(n):
        if nin[s] > 0:
            size[nx[s]] = size.get(nx[s], 0) + int(nin[s])

    def q(w):
        return int(np.int8(np.clip(np.float32(w) / np.float32(scale) + np.float32(zp), -128, 127)))

    e = 0
    for i in range(m):
        for j in range(i, m):
            k = nx[i]
            if nx[j] == k and term(k) and size.get(k, 0) > 0:
                v = 0
                if nin[j] > 0:
                    v += q(np.float32(nin[j]) / np.float32(size[k]))
                if i != j and nin[i] > 0:
                    v += q(np.float32(nin[i]) / np.float32(size[k]))
                out[e] = v
            e += 1
    return (out % 256).astype(np.uint8).view(np.int8)


@pytest.mark.parametrize("seed,scale,zp,n_real", [(1, 1 / 127.0, 0.0, 0), (2, 0.004, -20.0, 0), (3, 0.02, 3.0, 41)])
def test_tree_upper_i8_matches_pairwise_brute_force(seed, scale, zp, n_real):
    rng = np.random.default_rng(seed)
    n, nnode = 64, 7
    ns = np.where(rng.random(nnode) < 0.7, -1, 1).astype(np.int32)
    nx = rng.integers(-1, nnode + 1, n).astype(np.int32)
    nin = np.bincount(rng.integers(0, n, n), minlength=n).astype(np.int32)
    got = O.tree_upper(O.FMT_I8, ns, nx, nin, scale=np.float32(scale), zp=np.float32(zp), n_real=n_real)
    assert np.array_equal(got, i8_pair_brute(ns, nx, nin, scale, zp, n_real))


def test_tree_upper_n_real_is_the_leading_block():
    rng = np.random.default_rng(9)
    n, nnode, m = 90, 5, 61
    ns = -np.ones(nnode, np.int32)
    nx = rng.integers(0, nnode, n).astype(np.int32)
    nin = np.bincount(rng.integers(0, n, n), minlength=n).astype(np.int32)
    for fmt in (O.FMT_F16, O.FMT_I8):
        full = tri_dense(O.tree_upper(fmt, ns, nx, nin, casewise=True, scale=0.01).astype(np.float64), n)
        part = tri_dense(O.tree_upper(fmt, ns, nx, nin, casewise=True, scale=0.01, n_real=m)
                         .astype(np.float64), m)
        assert np.array_equal(full[:m, :m], part)


def test_rfgap_tree_upper_is_twice_single_tree_rfgap():
    """With one tree, cpu_proximity_rfgap (pinned above) gives
    (C_ij + C_ji)/2 for i != j, C_ij = nin[j]/size for OOB i and in-bag j of
    one node; the per-tree triangle holds C_ij for i <= j."""
    g = np.load(os.path.join(GOLD, "rfgap_small.npz"))
    nin, nx = g["nin"].astype(np.int32), g["nodextr"].astype(np.int32)
    n = nin.shape[1]
    for k in range(0, nin.shape[0], 5):
        dense = O.rfgap(nin[k:k + 1], nx[k:k + 1])
        want = np.triu(2 * dense, 1) * (nin[k] == 0)[:, None]
        got = tri_dense(O.rfgap_tree_upper(nin[k], nx[k]).view(np.float16).astype(np.float64), n)
        assert np.array_equal(got > 0, want > 0)
        assert np.abs(got - want).max() <= 2.0 ** -11 * max(want.max(), 1e-30)


# ---- QuantizationDispatcher::launch_proximity_kernel ---------------------------

def terminal_csr(ns, nx):
    """ndbegin / npcase of the terminal ordinals (src/rf_proximity.cpp:110-171)."""
    xb = O.terminal_leaf(ns, nx)
    nterm = int((np.asarray(ns) == -1).sum())
    cnt = np.bincount(xb[xb >= 0], minlength=nterm)
    beg = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
    pc = np.concatenate([np.flatnonzero(xb == k) for k in range(nterm)] + [np.zeros(0, np.int64)]).astype(np.int32)
    return xb, beg, pc


@pytest.mark.parametrize("seed", [4, 5])
def test_dispatch_prox_levels(seed):
    """FP32 level: rows of OOB samples equal the compiled reference's casewise
    cpu_proximity (n <= kk); every entry equals a pair-by-pair brute force.
    The other levels are the reference converters of the float weight."""
    rng = np.random.default_rng(seed)
    n, nnode = 97, 9
    ns = np.where(rng.random(nnode) < 0.7, -1, 1).astype(np.int32)
    nx = rng.integers(-1, nnode + 1, n).astype(np.int32)
    nin = np.bincount(rng.integers(0, n, n), minlength=n).astype(np.int32)
    xb, beg, pc = terminal_csr(ns, nx)
    D = O.dispatch_prox(0, xb, nin, beg, pc)
    size = np.array([nin[(xb == k) & (nin > 0)].sum() for k in range(len(beg) - 1)], np.int64)
    want = np.zeros((n, n))
    for a in range(n):
        for b in range(a, n):
            if xb[a] >= 0 and xb[a] == xb[b] and nin[b] > 0 and size[xb[a]] > 0:
                want[a, b] = nin[b] / size[xb[a]]
    assert np.array_equal(D, want)
    if O.ref_available():
        R = compiled_reference()
        R.ref_set_config(1, 0, 2)
        C = np.zeros((n, n), order="F")
        R.ref_cpu_proximity(ns, nx, nin, n, nnode, C.reshape(-1, order="F"))
        oob = nin == 0
        up = np.triu(np.ones((n, n), bool))
        assert np.array_equal(D[oob][up[oob]], C[oob][up[oob]])
        assert C[oob].any()
    hit = want > 0
    w32 = (np.float32(1) * nin[None, :].repeat(n, 0)).astype(np.float32)
    w32 = np.where(hit, w32 / np.where(xb >= 0, size[xb], 1).astype(np.float32)[:, None], np.float32(0))
    f16 = O.dispatch_prox(1, xb, nin, beg, pc)
    assert np.array_equal(f16, np.where(hit, w32.astype(np.float16).view(np.uint16), 0))
    i8 = O.dispatch_prox(2, xb, nin, beg, pc)
    q = np.clip(w32 / np.float32(1.0 / 127.0), -128, 127).astype(np.int8)
    assert np.array_equal(i8, np.where(hit, q, 0))
    nf = O.dispatch_prox(3, xb, nin, beg, pc)
    assert np.array_equal(nf, np.where(hit, np.minimum(7, np.floor(w32.astype(np.float64) * 7 + 0.5)), 0))


# ---- pair proximity and outlier scores ---------------------------------------

def test_pair_proximity_is_oob_match_fraction():
    rng = np.random.default_rng(21)
    n, t, nleaf = 120, 37, 5
    leaf = rng.integers(-1, nleaf, (t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.4).astype(np.uint8)
    oob[:, 3] = 0
    for i, j in [(0, 1), (5, 5), (17, 90), (3, 4), (119, 0), (-1, 2), (2, 120)]:
        got = O.pair_proximity(leaf, oob, nleaf, i, j)
        if not (0 <= i < n and 0 <= j < n) or oob[:, i].sum() == 0:
            assert got == 0.0
            continue
        m = int((oob[:, i].astype(bool) & (leaf[:, i] == leaf[:, j]) & (leaf[:, i] >= 0)).sum())
        assert got == np.float32(m) / np.float32(oob[:, i].sum())


def test_outlier_raw_equals_dense_cooccurrence():
    """raw = numerator / sum_j (C_ij / T)^2 with C the all-trees co-occurrence
    matrix taken as a dense one-hot product (an independent route)."""
    rng = np.random.default_rng(22)
    n, t, nleaf = 300, 23, 6
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    leaf[0, :40] = np.arange(40) % nleaf
    C = np.zeros((n, n))
    for k in range(t):
        A = np.zeros((n, nleaf))
        A[np.arange(n), leaf[k]] = 1
        C += A @ A.T
    np.fill_diagonal(C, 0)
    p = (C.astype(np.float32) / np.float32(t))
    s = (p.astype(np.float32) * p.astype(np.float32)).astype(np.float64).sum(axis=1).astype(np.float32)
    want = np.float32(n - 1) / s
    got = O.outlier_raw(leaf, nleaf, np.ascontiguousarray(leaf.T), exclude=np.arange(n, dtype=np.int32),
                        numerator=float(n - 1), isolated=float(n) * 1e10)
    assert np.allclose(got, want, rtol=1e-6, atol=0)
    # anchors: a subset as the reference set, excluding a query's own anchor
    anchors = np.array([3, 50, 77, 200], np.int32)
    ex = np.full(n, -1, np.int32)
    ex[anchors] = np.arange(len(anchors))
    ga = O.outlier_raw(np.ascontiguousarray(leaf[:, anchors]), nleaf, np.ascontiguousarray(leaf.T), exclude=ex,
                       numerator=4.0, isolated=4e10)
    pa = p[:, anchors]
    sa = (pa * pa).astype(np.float64).sum(axis=1).astype(np.float32)
    wa = np.where(sa > np.float32(1e-10), np.float32(4.0) / np.maximum(sa, np.float32(1e-30)), np.float32(4e10))
    assert np.allclose(ga, wa, rtol=1e-6, atol=0)


def test_outlier_normalize_reference_median_rule():
    """median = sorted[size/2] (upper median), MAD likewise, 1 below 1e-10."""
    got = O.outlier_normalize(np.array([5, 1, 3, 2, 4], np.float32))
    assert np.array_equal(got, np.array([2, -2, 0, -1, 1], np.float32))
    got = O.outlier_normalize(np.array([1, 2, 3, 4], np.float32))           # median 3, MAD 1
    assert np.array_equal(got, np.array([-2, -1, 0, 1], np.float32))
    got = O.outlier_normalize(np.array([7, 7, 7, 9], np.float32))           # MAD 0 -> 1
    assert np.array_equal(got, np.array([0, 0, 0, 2], np.float32))
    raw = np.array([10, 1, 20, 2, 30, 3], np.float32)
    cls = np.array([1, 0, 1, 0, 1, 0], np.int32)                            # medians 20 / 2, MADs 10 / 1
    got = O.outlier_normalize(raw, cls)
    assert np.array_equal(got, np.array([-1, -1, 0, 0, 1, 1], np.float32))


# ---- leaf assignments on a forest ---------------------------------------------

def random_forest_arrays(rng, t, maxnode, cat, maxcat):
    mdim = len(cat)
    ns = -np.ones((t, maxnode), np.int32)
    bv = np.zeros((t, maxnode), np.int32)
    sp = np.zeros((t, maxnode), np.float32)
    tm = np.zeros((t, maxnode, 2), np.int32)
    cg = rng.integers(0, 2, (t, maxnode, maxcat)).astype(np.int32)
    for k in range(t):
        nodes, queue = 1, [0]
        while queue:
            v = queue.pop(0)
            bv[k, v] = rng.integers(0, mdim)
            sp[k, v] = np.float32(rng.standard_normal() * 0.8)
            if nodes + 2 <= maxnode and rng.random() < 0.8:
                ns[k, v] = 2 if rng.random() < 0.05 else 1
                tm[k, v] = (nodes, nodes + 1)
                queue += [nodes, nodes + 1]
                nodes += 2
    return dict(nodestatus=ns, bestvar=bv, xbestsplit=sp, treemap=tm, catgoleft=cg, cat=np.asarray(cat, np.int32))


def random_features(rng, n, cat):
    X = rng.standard_normal((n, len(cat))).astype(np.float32)
    for v, c in enumerate(cat):
        if c > 1:   # category codes with fractions and out-of-range values
            X[:, v] = (rng.integers(-1, c + 2, n) + rng.choice([0.0, 0.3, 0.5, 0.7, -0.2], n)).astype(np.float32)
    return X


def test_forest_leaves_oob_walk_equals_compiled_testreebag():
    Rf = compiled_reference()
    rng = np.random.default_rng(61)
    cat, maxcat, t, n, maxnode = [1, 1, 3, 5, 2, 1], 5, 12, 400, 41
    f = random_forest_arrays(rng, t, maxnode, cat, maxcat)
    X = random_features(rng, n, cat)
    nin = (rng.random((t, n)) < 0.6).astype(np.int32) * rng.integers(1, 3, (t, n)).astype(np.int32)
    got = O.forest_leaves(1, f, X, nin)
    Rf.ref_cpu_testreebag.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_int32] * 4 + [ctypes.c_void_p]
    for k in range(t):
        nodextr = np.empty(n, np.int32)
        Rf.ref_cpu_testreebag(X.ctypes.data, np.ascontiguousarray(f["xbestsplit"][k]).ctypes.data,
                              np.ascontiguousarray(nin[k]).ctypes.data,
                              np.ascontiguousarray(f["treemap"][k]).ctypes.data,
                              np.ascontiguousarray(f["bestvar"][k]).ctypes.data, f["cat"].ctypes.data,
                              np.ascontiguousarray(f["nodestatus"][k]).ctypes.data,
                              np.ascontiguousarray(f["catgoleft"][k]).ctypes.data, n, len(cat), maxnode, maxcat,
                              nodextr.ctypes.data)
        oob = nin[k] == 0
        assert np.array_equal(got[k][oob], nodextr[oob]), k
        assert (f["nodestatus"][k][got[k][oob]] != 1).all()


def sklearn_forest(rng, t, n, mdim):
    from sklearn.tree import DecisionTreeRegressor

    X = rng.standard_normal((n, mdim)).astype(np.float32)
    y = np.sin(X[:, 0]) + X[:, 1] * X[:, 2] + 0.1 * rng.standard_normal(n)
    trees = [DecisionTreeRegressor(max_depth=7, random_state=k).fit(X[rng.integers(0, n, n)], y)
             for k in range(t)]
    maxnode = max(tr.tree_.node_count for tr in trees)
    ns = -np.ones((t, maxnode), np.int32)
    bv = np.zeros((t, maxnode), np.int32)
    sp = np.zeros((t, maxnode), np.float32)
    tm = np.zeros((t, maxnode, 2), np.int32)
    for k, tr in enumerate(trees):
        s = tr.tree_
        m = s.node_count
        split = s.children_left >= 0
        ns[k, :m] = np.where(split, 1, -1)
        bv[k, :m] = np.where(split, s.feature, 0)
        thr = s.threshold.astype(np.float32)          # largest float32 <= the double threshold:
        thr = np.where(thr.astype(np.float64) > s.threshold, np.nextafter(thr, np.float32(-np.inf)), thr)
        sp[k, :m] = np.where(split, thr, 0)           # x <= thr32 iff x <= thr for float32 x
        tm[k, :m, 0] = np.where(split, s.children_left, 0)
        tm[k, :m, 1] = np.where(split, s.children_right, 0)
    return trees, dict(nodestatus=ns, bestvar=bv, xbestsplit=sp, treemap=tm, catgoleft=None, cat=None), X


def test_forest_leaves_numeric_walks_equal_sklearn_apply():
    """On numeric trees all three walks reach the leaf sklearn's apply()
    reports (its own traversal, x <= threshold goes left)."""
    rng = np.random.default_rng(62)
    trees, f, X = sklearn_forest(rng, 6, 700, 5)
    Xq = rng.standard_normal((300, 5)).astype(np.float32)
    want = np.stack([tr.apply(Xq) for tr in trees]).astype(np.int32)
    assert np.array_equal(O.forest_leaves(0, f, Xq), want)
    for nin in (np.ones((6, 300), np.int32), np.zeros((6, 300), np.int32)):
        assert np.array_equal(O.forest_leaves(1, f, Xq, nin), want)


def test_forest_leaves_categorical_rules():
    """One categorical split at the root: predict and find_terminal_node use
    (int)(x + 0.5), testreebag uses (int)x and sends invalid codes right;
    find_terminal_node returns 0 for an invalid code, predict stays at 0."""
    cat = np.array([4], np.int32)
    ns = np.array([[1, -1, -1]], np.int32)
    f = dict(nodestatus=ns, bestvar=np.zeros((1, 3), np.int32), xbestsplit=np.zeros((1, 3), np.float32),
             treemap=np.array([[[1, 2], [0, 0], [0, 0]]], np.int32),
             catgoleft=np.array([[[1, 0, 1, 0], [0] * 4, [0] * 4]], np.int32), cat=cat)
    x = np.array([[0.0], [0.4], [0.6], [1.49], [2.5], [3.6], [-0.6], [-0.4], [4.2]], np.float32)
    rnd = [0, 0, 1, 1, 3, 4, 0, 0, 4]           # (int)(x + 0.5), truncation toward 0
    trc = [0, 0, 0, 1, 2, 3, 0, 0, 4]           # (int)x
    pred = O.forest_leaves(0, f, x)[0]
    inbag = O.forest_leaves(1, f, x, np.ones((1, len(x)), np.int32))[0]
    oob = O.forest_leaves(1, f, x, np.zeros((1, len(x)), np.int32))[0]
    go = lambda c: 1 if f["catgoleft"][0, 0, c] == 1 else 2  # noqa: E731
    assert list(pred) == [go(c) if 0 <= c < 4 else 0 for c in rnd]
    assert list(inbag) == [go(c) if 0 <= c < 4 else 0 for c in rnd]
    assert list(oob) == [go(c) if 0 <= c < 4 else 2 for c in trc]


def test_forest_leaves_feed_the_reference_proximity():
    """Training leaves as nodextr, with non-terminal nodes excluded, give the
    compiled reference's cpu_proximity + cpu_finishprox through the
    triangle restatement: the producer composes with the proximity path."""
    Rf = compiled_reference()
    rng = np.random.default_rng(63)
    trees, f, X = sklearn_forest(rng, 8, 300, 5)
    t, maxnode = f["nodestatus"].shape
    n = X.shape[0]
    nin = np.stack([np.bincount(rng.integers(0, n, n), minlength=n) for _ in range(t)]).astype(np.int32)
    leaf = O.forest_leaves(1, f, X, nin)
    Rf.ref_set_config(0, 0, 2)
    pr = np.zeros((n, n), order="F")
    for k in range(t):
        Rf.ref_cpu_proximity(np.ascontiguousarray(f["nodestatus"][k]), np.ascontiguousarray(leaf[k]), nin[k], n,
                             maxnode, pr.reshape(-1, order="F"))
    nout = (nin == 0).sum(axis=0).astype(np.int32)
    ps = np.zeros((n, n), order="F")
    Rf.ref_cpu_finishprox(n, nout, pr.reshape(-1, order="F"), ps.reshape(-1, order="F"))
    term = np.where(np.take_along_axis(f["nodestatus"], leaf, axis=1) == -1, leaf, -1).astype(np.int32)
    got = O.upper_rows(term, (nin == 0).astype(np.uint8), maxnode, O.FMT_F32)
    assert np.array_equal(got, ps[np.triu_indices(n)].astype(np.float32))


def both_oob_dense(leaf, oob, nleaf):
    """Independent numpy evaluation of the both-OOB proximity: num and den as
    (N, N) arrays from broadcast comparisons over the trees."""
    valid = (leaf >= 0) & (leaf < nleaf)
    o = oob.astype(bool)
    both = o[:, :, None] & o[:, None, :]                       # (T, N, N)
    same = (leaf[:, :, None] == leaf[:, None, :]) & valid[:, :, None] & valid[:, None, :]
    return (both & same).sum(0), both.sum(0)


@pytest.mark.parametrize("n,t,nleaf,r0,r1", [(1, 3, 2, 0, 1), (7, 33, 3, 0, 7), (60, 45, 5, 0, 60),
                                             (61, 64, 4, 13, 50)])
def test_both_oob_matches_independent_evaluation(n, t, nleaf, r0, r1):
    rng = np.random.default_rng(n * 7 + t)
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    leaf[rng.random((t, n)) < 0.05] = -1
    oob = (rng.random((t, n)) < 0.4).astype(np.uint8)
    if n > 3:
        oob[:, 2] = 0            # never OOB: den 0 with everyone
        oob[:, 3] = 1            # always OOB
    num, den = both_oob_dense(leaf, oob, nleaf)
    iu = np.triu_indices(n)
    keep = (iu[0] >= r0) & (iu[0] < r1)
    i, j = iu[0][keep], iu[1][keep]
    want_u16 = np.where(i == j, 0, num[i, j]).astype(np.uint16)
    with np.errstate(invalid="ignore", divide="ignore"):
        p = np.where(den[i, j] > 0, num[i, j].astype(np.float32) / den[i, j].astype(np.float32), np.float32(0))
    want_f32 = np.where(i == j, np.float32(1), p).astype(np.float32)
    assert np.array_equal(O.both_oob_rows(leaf, oob, nleaf, O.FMT_U16, r0, r1), want_u16)
    assert np.array_equal(O.both_oob_rows(leaf, oob, nleaf, O.FMT_F32, r0, r1), want_f32)


def test_both_oob_hand_example():
    """Three samples, four trees, worked by hand: samples 0 and 1 are both OOB
    in trees 0, 1, 3 and share a leaf in trees 0 and 3 -> 2/3; sample 2 is OOB
    only in tree 2, alone -> 0 with both."""
    leaf = np.array([[0, 0, 1], [1, 0, 1], [0, 1, 0], [2, 2, 2]], np.int32)
    oob = np.array([[1, 1, 0], [1, 1, 0], [0, 0, 1], [1, 1, 0]], np.uint8)
    got = O.both_oob_rows(leaf, oob, 3, O.FMT_F32)
    want = np.array([1.0, np.float32(2) / np.float32(3), 0.0, 1.0, 0.0, 1.0], np.float32)
    assert np.array_equal(got, want)
    assert np.array_equal(O.both_oob_rows(leaf, oob, 3, O.FMT_U16), np.array([0, 2, 0, 0, 0, 0], np.uint16))


def test_pair_total_closed_form_matches_the_oracle_triangle():
    """The closed form behind the full-size triangle check (sum of U over
    i < j = sum over trees and leaves of #OOB x #in-bag) against the
    oracle's U16 triangle, with invalid labels mixed in."""
    from closed_forms import pair_total

    rng = np.random.default_rng(91)
    n, t, nleaf = 300, 40, 7
    leaf = rng.integers(-1, nleaf + 1, size=(t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.4).astype(np.uint8)
    tri = O.upper_rows(leaf, oob, nleaf, O.FMT_U16)
    assert int(tri.astype(np.int64).sum()) == pair_total(leaf, oob, nleaf)


def symmetric_row_sums_np(tri, n):
    """Per sample, the sum of U over its row and column of the packed upper
    triangle (the diagonal, 0 in U16, taken once from each side)."""
    out = np.zeros(n, dtype=np.int64)
    e = 0
    for i in range(n):
        row = tri[e:e + n - i].astype(np.int64)
        out[i] += row.sum()
        out[i:] += row
        e += n - i
    return out


def test_row_pair_counts_closed_form_matches_the_oracle_triangle():
    """The per-sample closed form behind the full-size row-sum check (sum of
    U_ij over j != i = sum over trees of the size of i's opposite bucket)
    against the oracle's U16 triangle, invalid labels included; a count
    moved to another column of the same row keeps the total but breaks the
    row sums, so the check catches what pair_total cannot."""
    from closed_forms import row_pair_counts

    rng = np.random.default_rng(92)
    n, t, nleaf = 300, 40, 7
    leaf = rng.integers(-1, nleaf + 1, size=(t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.4).astype(np.uint8)
    tri = O.upper_rows(leaf, oob, nleaf, O.FMT_U16)
    want = row_pair_counts(leaf, oob, nleaf)
    assert np.array_equal(symmetric_row_sums_np(tri, n), want)
    # the torch version the full-size GPU tests use, run here on the CPU
    import torch
    from tri_sums import symmetric_row_sums

    got = symmetric_row_sums(torch.from_numpy(tri.view(np.int16)), n, block=37).numpy()
    assert np.array_equal(got, want)
    # a planted mistake: one count moved within row 0 (columns 5 -> 9)
    bad = tri.astype(np.int64).copy()
    bad[5] -= 1
    bad[9] += 1
    assert int(bad.sum()) == int(tri.astype(np.int64).sum())
    assert not np.array_equal(symmetric_row_sums_np(bad, n), want)
