"""Top-K retrieval, its scores, pair proximity and outlier sums: the
library's kernels run on the CPU by the emulator (tests/emu, script mode),
through the C ABI, against the oracle's brute force.  Same bar as the GPU
tests: identical indices and counts (ties by the lower reference index),
float scores equal, raw outlier sums within 1e-6.  Sizes are cut to what
the emulation runs in seconds; the segment shapes the kernels choose from N
and T (16-bit segments, 8-bit segments with the byte-sum check and their
recount) are each reached."""
import numpy as np
import pytest

import oracle as O
from emu_session import CTX, EmuScript
from test_emu_cpu import pack_words


def topk_script(s, ref, nleaf, qs, k, exclude_base=-1, oob_words=None, positive_only=0, layout="query"):
    """rfxp_set_reference + rfxp_topk; qs is Q x T (layout 'query') or the
    T x Q tree-major matrix (layout 'tree')."""
    t, n = ref.shape
    q = qs.shape[0] if layout == "query" else qs.shape[1]
    si, st = (t, 1) if layout == "query" else (1, q)
    r = s.dev(ref.astype(np.int32))
    qb = s.dev(qs.astype(np.int32))
    ob = s.dev(oob_words) if oob_words is not None else None
    idx, cnt = s.out(4 * q * k), s.out(2 * q * k)
    s.call("rfxp_set_reference", CTX, r, 1, n, n, t, nleaf)
    s.call("rfxp_topk", CTX, qb, si, st, q, ob, oob_words.shape[1] if ob is not None else 0, exclude_base, k,
           positive_only, idx, cnt)
    return idx, cnt


@pytest.mark.parametrize("n,t,nleaf,q,k", [(5, 3, 2, 4, 3),          # K > N
                                           (1000, 40, 7, 9, 20),
                                           (2100, 16, 300, 5, 64),
                                           (40000, 24, 50, 3, 20),   # 16-bit segments
                                           (70001, 12, 9, 3, 1),     # 8-bit segments
                                           # K > 32 on 8-bit segments: candidates gathered with the
                                           # lanes that hold none masked off (a ballot prefix in a branch)
                                           (79353, 17, 64, 1, 42), (60434, 17, 1000, 4, 56)])
def test_topk_all_trees(emu_driver, tmp_path, n, t, nleaf, q, k):
    rng = np.random.default_rng(n + t + q)
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    qs = rng.integers(0, nleaf, size=(q, t), dtype=np.int32)
    qs[0] = ref[:, n // 2]
    s = EmuScript(emu_driver)
    idx, cnt = topk_script(s, ref, nleaf, qs, k)
    assert s.run(tmp_path) == [0, 0]
    want_i, want_c = O.topk_all(ref, qs, k, nleaf=nleaf)
    if k > n:
        want_i[:, n:], want_c[:, n:] = -1, 0
    assert np.array_equal(cnt.array(np.uint16, (q, k)), want_c)
    assert np.array_equal(idx.array(np.int32, (q, k)), want_i)


def test_topk_wrapped_8bit_counts_and_exclusion(emu_driver, tmp_path):
    """8-bit segments with T = 300 > 255 (the byte-sum check): planted copies
    of the queries around block and segment boundaries reach counts of 300
    and 280 that wrap 8 bits and take the 16-bit recount; one planted copy
    excluded; the raw outlier sums over the same segments."""
    rng = np.random.default_rng(31)
    n, t, nleaf, q, k = 70_001, 300, 40, 4, 12
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    qs = rng.integers(0, nleaf, size=(q, t), dtype=np.int32)
    for pos in (1000, 32767, 65536, 70000):
        ref[:, pos] = qs[0]
    near = qs[1].copy()
    near[:20] = (near[:20] + 1) % nleaf            # 280 of 300 trees match
    ref[:, 40000] = near
    ref[:, 65535] = qs[2]
    ref[:, 32768] = qs[3]
    s = EmuScript(emu_driver)
    idx, cnt = topk_script(s, ref, nleaf, qs, k)
    qb = s.dev(qs)
    idx2, cnt2 = s.out(4 * q * k), s.out(2 * q * k)
    s.call("rfxp_topk", CTX, qb, t, 1, q, None, 0, 65535, k, 0, idx2, cnt2)   # query 0 may not return 65535
    raw = s.out(4 * q)
    s.call("rfxp_outlier_raw", CTX, qb, t, 1, q, 32767, None, float(n - 1), n * 1e10, raw)
    assert s.run(tmp_path) == [0] * 4
    want_i, want_c = O.topk_all(ref, qs, k, nleaf=nleaf)
    assert np.array_equal(cnt.array(np.uint16, (q, k)), want_c)
    assert np.array_equal(idx.array(np.int32, (q, k)), want_i)
    assert cnt.array(np.uint16, (q, k))[0, :4].tolist() == [t] * 4 and want_c[1, 0] == 280
    want_i, want_c = O.topk_all(ref, qs, k, exclude=np.arange(65535, 65535 + q, dtype=np.int32), nleaf=nleaf)
    assert np.array_equal(cnt2.array(np.uint16, (q, k)), want_c)
    assert np.array_equal(idx2.array(np.int32, (q, k)), want_i)
    want = O.outlier_raw(ref, nleaf, qs, exclude=np.arange(32767, 32767 + q, dtype=np.int32),
                         numerator=float(n - 1), isolated=n * 1e10)
    assert np.allclose(raw.array(np.float32), want, rtol=1e-6, atol=0)


def test_topk_invalid_labels_and_self_exclusion(emu_driver, tmp_path):
    """Labels -1, -2 and nleaf + 3 never match, also where query and
    reference hold the same one (training samples queried tree-major, each
    excluding itself)."""
    rng = np.random.default_rng(5)
    n, t, nleaf, q, k = 3000, 20, 11, 10, 30
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    ref[rng.random((t, n)) < 0.1] = -1
    ref[rng.random((t, n)) < 0.05] = nleaf + 3
    qs = rng.integers(0, nleaf, size=(q, t), dtype=np.int32)
    qs[rng.random((q, t)) < 0.2] = -2
    s = EmuScript(emu_driver)
    idx, cnt = topk_script(s, ref, nleaf, qs, k)
    tq = np.ascontiguousarray(ref[:, 100:140])     # training samples 100..139, tree-major
    idx2, cnt2 = s.out(4 * 40 * 12), s.out(2 * 40 * 12)
    s.call("rfxp_topk", CTX, s.dev(tq), 1, 40, 40, None, 0, 100, 12, 0, idx2, cnt2)
    assert s.run(tmp_path) == [0, 0, 0]
    want_i, want_c = O.topk_all(ref, qs, k, nleaf=nleaf)
    assert np.array_equal(cnt.array(np.uint16, (q, k)), want_c)
    assert np.array_equal(idx.array(np.int32, (q, k)), want_i)
    want_i, want_c = O.topk_all(ref, np.ascontiguousarray(tq.T), 12, exclude=np.arange(100, 140, dtype=np.int32),
                                nleaf=nleaf)
    assert np.array_equal(cnt2.array(np.uint16, (40, 12)), want_c)
    assert np.array_equal(idx2.array(np.int32, (40, 12)), want_i)


def test_topk_oob_queries_and_scores(emu_driver, tmp_path):
    """OOB queries of the training samples against their own forest (only
    trees where the query is OOB, itself excluded, counts > 0), and the
    float scores of both query kinds."""
    rng = np.random.default_rng(13)
    n, t, nleaf, k = 600, 45, 7, 9
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    oob[:, 7] = 0                                   # never OOB: no results
    words = pack_words(oob)
    s = EmuScript(emu_driver)
    idx, cnt = topk_script(s, leaf, nleaf, leaf, k, exclude_base=0, oob_words=words, positive_only=1,
                           layout="tree")
    wb = s.dev(words)
    sc = s.out(4 * n * k)
    s.call("rfxp_topk_scores", CTX, wb, words.shape[1], n, t, k, idx, cnt, sc)
    qs = rng.integers(0, nleaf, size=(30, t), dtype=np.int32)
    qb = s.dev(qs)
    idx2, cnt2, sc2 = s.out(4 * 30 * k), s.out(2 * 30 * k), s.out(4 * 30 * k)
    s.call("rfxp_topk", CTX, qb, t, 1, 30, None, 0, -1, k, 0, idx2, cnt2)
    s.call("rfxp_topk_scores", CTX, None, 0, 30, t, k, idx2, cnt2, sc2)
    assert s.run(tmp_path) == [0] * 5
    I, C, S = idx.array(np.int32, (n, k)), cnt.array(np.uint16, (n, k)), sc.array(np.float32, (n, k))
    for q in range(n):
        wi, wc, ws = O.topk_oob(leaf, oob, q, k, nleaf=nleaf)
        m = len(wi)
        assert np.array_equal(I[q, :m], wi) and np.array_equal(C[q, :m], wc), q
        assert np.array_equal(S[q, :m], ws) and (S[q, m:] == 0).all(), q
        assert (I[q, m:] == -1).all() and (C[q, m:] == 0).all(), q
    c2 = cnt2.array(np.uint16, (30, k)).astype(np.float32)
    assert np.array_equal(sc2.array(np.float32, (30, k)), c2 / np.float32(t))


def test_pair_proximity(emu_driver, tmp_path):
    rng = np.random.default_rng(32)
    n, t, nleaf = 1500, 130, 9
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    leaf[rng.random((t, n)) < 0.05] = -1
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    oob[:, 17] = 0
    words = pack_words(oob)
    pi = rng.integers(-2, n + 2, 400).astype(np.int64)
    pj = rng.integers(-2, n + 2, 400).astype(np.int64)
    pi[:5], pj[:5] = [17, 4, 9, 9, 0], [3, 4, 9, 17, n - 1]
    s = EmuScript(emu_driver)
    outs = []
    for layout in ("tree", "sample"):
        lf = leaf if layout == "tree" else np.ascontiguousarray(leaf.T)
        si, st = (1, n) if layout == "tree" else (t, 1)
        o = s.out(4 * len(pi))
        s.call("rfxp_pair_proximity", CTX, s.dev(lf), si, st, s.dev(words), words.shape[1], n, t, nleaf,
               s.dev(pi), s.dev(pj), len(pi), o)
        outs.append(o)
    assert s.run(tmp_path) == [0, 0]
    want = np.array([O.pair_proximity(leaf, oob, nleaf, a, b) for a, b in zip(pi, pj)], np.float32)
    for o in outs:
        assert np.array_equal(o.array(np.float32), want)


def test_outlier_full_and_anchor_modes(emu_driver, tmp_path):
    rng = np.random.default_rng(33)
    n, t, nleaf = 800, 60, 25
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    s = EmuScript(emu_driver)
    lb = s.dev(leaf)
    raw = s.out(4 * n)
    s.call("rfxp_set_reference", CTX, lb, 1, n, n, t, nleaf)
    s.call("rfxp_outlier_raw", CTX, lb, 1, n, n, 0, None, float(n - 1), float(n) * 1e10, raw)
    anchors = np.sort(rng.choice(n, 100, replace=False)).astype(np.int64)
    ex = np.full(n, -1, np.int32)
    ex[anchors] = np.arange(len(anchors))
    aleaf = np.ascontiguousarray(leaf[:, anchors])
    raw2 = s.out(4 * n)
    s.call("rfxp_set_reference", CTX, s.dev(aleaf), 1, len(anchors), len(anchors), t, nleaf)
    s.call("rfxp_outlier_raw", CTX, lb, 1, n, n, -1, s.dev(ex), 100.0, 100.0 * 1e10, raw2)
    assert s.run(tmp_path) == [0] * 4
    want = O.outlier_raw(leaf, nleaf, np.ascontiguousarray(leaf.T), exclude=np.arange(n, dtype=np.int32),
                         numerator=float(n - 1), isolated=float(n) * 1e10)
    assert np.allclose(raw.array(np.float32), want, rtol=1e-6, atol=0)
    want = O.outlier_raw(aleaf, nleaf, np.ascontiguousarray(leaf.T), exclude=ex, numerator=100.0,
                         isolated=100.0 * 1e10)
    assert np.allclose(raw2.array(np.float32), want, rtol=1e-6, atol=0)
