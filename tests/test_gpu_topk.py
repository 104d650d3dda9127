"""GPU parity of top-K similarity retrieval (rfxp_set_reference + rfxp_topk)
against the CPU oracle's brute-force restatements, which tests/test_oracle.py
pins to an independent brute force.  Bar: identical indices and counts,
ties broken by the lower reference index."""
import numpy as np
import pytest

import oracle as O
import rfxprox as R

pytestmark = pytest.mark.gpu


def dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def run_topk(ctx, ref_tn, nleaf, q_qt, k, **kw):
    t, n = ref_tn.shape
    ctx.set_reference(dev(ref_tn.astype(np.int32)), n, t, nleaf)
    idx, cnt = ctx.topk(dev(q_qt.astype(np.int32)), k, **kw)
    return idx.cpu().numpy(), cnt.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("n,t,nleaf,q,k", [(5, 3, 2, 4, 3), (1000, 40, 7, 33, 20), (2100, 16, 300, 17, 64),
                                           (40000, 24, 50, 12, 20), (70001, 12, 9, 9, 1)])
def test_all_trees_topk_matches_oracle(gpu_ctx, n, t, nleaf, q, k):
    rng = np.random.default_rng(n + t + q)
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    qs = rng.integers(0, nleaf, size=(q, t), dtype=np.int32)
    qs[0] = ref[:, n // 2]            # a query identical to one reference: count T
    got_i, got_c = run_topk(gpu_ctx, ref, nleaf, qs, k)
    want_i, want_c = O.topk_all(ref, qs, k)
    if k > n:
        want_i[:, n:], want_c[:, n:] = -1, 0
    assert np.array_equal(got_c, want_c)
    assert np.array_equal(got_i, want_i)


def test_eight_bit_segments_with_wrapped_counts(gpu_ctx):
    """Reference sets above 65536 samples with T <= 2048 are counted with 8-bit
    counters in segments of 131072 (four blocks of 32768); T = 300 > 255
    turns on the byte-sum check.  Copies of the queries planted in several
    blocks of a segment, on the two sides of block boundaries and of the
    segment boundary, and in the short last segment reach counts of 300 (and
    280 for a near copy), which wrap 8 bits and force the 16-bit recount,
    block by block; with and without the exclusion of one planted copy.  40
    leaves make runs of thousands of members (loads past the first 128).
    Outlier sums over the same segments too."""
    rng = np.random.default_rng(31)
    n, t, nleaf, q, k = 140_000, 300, 40, 6, 20
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    qs = rng.integers(0, nleaf, size=(q, t), dtype=np.int32)
    for pos in (1000, 40000, 100000, 139999):
        ref[:, pos] = qs[0]
    for pos in (131071, 131072):
        ref[:, pos] = qs[1]
    for pos in (32767, 98304):
        ref[:, pos] = qs[2]
    near = qs[3].copy()
    near[:20] = (near[:20] + 1) % nleaf          # 280 of 300 trees match
    ref[:, 70000] = near
    ref[:, 65535] = qs[4]
    got_i, got_c = run_topk(gpu_ctx, ref, nleaf, qs, k)
    want_i, want_c = O.topk_all(ref, qs, k)
    assert np.array_equal(got_c, want_c) and np.array_equal(got_i, want_i)
    assert got_c[0, :4].tolist() == [t] * 4 and got_c[3, 0] == 280
    # exclude_base 40000: query 0 may not return its copy at 40000
    idx, cnt = gpu_ctx.topk(dev(qs), k, exclude_base=40000)
    want_i, want_c = O.topk_all(ref, qs, k, exclude=np.arange(40000, 40000 + q, dtype=np.int32))
    assert np.array_equal(cnt.cpu().numpy().view(np.uint16), want_c)
    assert np.array_equal(idx.cpu().numpy(), want_i)
    raw = gpu_ctx.outlier_raw(dev(qs), exclude_base=40000, numerator=float(n - 1), isolated=n * 1e10)
    want = O.outlier_raw(ref, nleaf, qs, exclude=np.arange(40000, 40000 + q, dtype=np.int32),
                         numerator=float(n - 1), isolated=n * 1e10)
    assert np.allclose(raw.cpu().numpy(), want, rtol=1e-6, atol=0)


@pytest.mark.parametrize("n,t,nleaf", [(70_000, 1100, 30),    # 8-bit, 3 of 4 blocks used, > 64 trees per wave
                                       (60_000, 400, 25),     # 8-bit segments of two blocks, counts wrap
                                       (40_000, 2100, 20)])   # above 2048 trees: 16-bit segments of 32768
def test_many_trees(gpu_ctx, n, t, nleaf):
    rng = np.random.default_rng(n + t)
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    qs = rng.integers(0, nleaf, size=(5, t), dtype=np.int32)
    ref[:, 33_000] = qs[0]       # counts of t wrap 8 bits
    ref[:, 65_535 if n > 65_535 else 32_767] = qs[1]
    got_i, got_c = run_topk(gpu_ctx, ref, nleaf, qs, 12)
    want_i, want_c = O.topk_all(ref, qs, 12)
    assert np.array_equal(got_c, want_c) and np.array_equal(got_i, want_i)
    assert got_c[0, 0] == t
    # outlier sums over the same segments (the wrapped ones recounted), one
    # planted copy excluded
    raw = gpu_ctx.outlier_raw(dev(qs), exclude_base=33_000, numerator=float(n - 1), isolated=n * 1e10)
    want = O.outlier_raw(ref, nleaf, qs, exclude=np.arange(33_000, 33_005, dtype=np.int32),
                         numerator=float(n - 1), isolated=n * 1e10)
    assert np.allclose(raw.cpu().numpy(), want, rtol=1e-6, atol=0)


def test_invalid_labels_never_match(gpu_ctx):
    rng = np.random.default_rng(5)
    n, t, nleaf, q, k = 3000, 20, 11, 10, 30
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    ref[rng.random((t, n)) < 0.1] = -1
    qs = rng.integers(0, nleaf, size=(q, t), dtype=np.int32)
    qs[rng.random((q, t)) < 0.2] = -2
    qs[:, 0] = ref[0, :q]                        # equal invalid labels (-1 and -1) are no match either
    got_i, got_c = run_topk(gpu_ctx, ref, nleaf, qs, k)
    want_i, want_c = O.topk_all(ref, qs, k, nleaf=nleaf)
    assert np.array_equal(got_c, want_c) and np.array_equal(got_i, want_i)


def test_exclude_self(gpu_ctx):
    rng = np.random.default_rng(8)
    n, t, nleaf, k = 900, 30, 6, 12
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    qs = np.ascontiguousarray(ref[:, 100:140].T)   # training samples 100..139 as queries
    got_i, got_c = run_topk(gpu_ctx, ref, nleaf, qs, k, exclude_base=100)
    want_i, want_c = O.topk_all(ref, qs, k, exclude=np.arange(100, 140, dtype=np.int32))
    assert np.array_equal(got_c, want_c) and np.array_equal(got_i, want_i)


@pytest.mark.parametrize("n,t,nleaf,k,nsample", [(1500, 60, 8, 10, None),
                                                 (70_000, 300, 40, 20, 25)])  # 8-bit, four blocks, wrap check
def test_oob_query_semantics(gpu_ctx, n, t, nleaf, k, nsample):
    """OOB queries of the training samples against their own forest: only
    the trees where the query is out-of-bag, itself excluded, counts > 0;
    every query (or a sample of them) against the oracle."""
    import torch

    rng = np.random.default_rng(13 + n)
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    oob[:, 7] = 0                                    # a sample never OOB: no results
    gpu_ctx.set_reference(dev(leaf), n, t, nleaf)
    words = R.pack_oob_bits(dev(oob).to(torch.bool))
    idx, cnt = gpu_ctx.topk(dev(leaf), k, layout="tree", oob_words=words, exclude_base=0,
                            positive_only=True)
    idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy().view(np.uint16)
    qs = range(n) if nsample is None else [7, 0, n - 1] + sorted(rng.choice(n, nsample, replace=False).tolist())
    for q in qs:
        wi, wc, _ = O.topk_oob(leaf, oob, q, k)
        m = len(wi)
        assert np.array_equal(idx[q, :m], wi) and np.array_equal(cnt[q, :m], wc), q
        assert (idx[q, m:] == -1).all() and (cnt[q, m:] == 0).all(), q


def test_c5_shape_sampled_queries(gpu_ctx):
    """Config C5 shape (N=1M references, T=500, 2048 leaves, uniform) with a
    few queries: the oracle's brute force costs Q*N*T compares."""
    import torch

    n, t, nleaf, q, k = 1_000_000, 500, 2048, 6, 20
    g = torch.Generator(device="cuda:0")
    g.manual_seed(20261201 + 5)
    ref = torch.randint(0, nleaf, (t, n), generator=g, device="cuda:0", dtype=torch.int32)
    qs = torch.randint(0, nleaf, (q, t), generator=g, device="cuda:0", dtype=torch.int32)
    qs[1] = ref[:, 123456]
    gpu_ctx.set_reference(ref, n, t, nleaf)
    idx, cnt = gpu_ctx.topk(qs, k)
    want_i, want_c = O.topk_all(ref.cpu().numpy(), qs.cpu().numpy(), k)
    assert np.array_equal(cnt.cpu().numpy().view(np.uint16), want_c)
    assert np.array_equal(idx.cpu().numpy(), want_i)
    assert idx[1, 0].item() == 123456 and cnt[1, 0].item() == t


def test_topk_rejects_bad_arguments(gpu_ctx):
    import ctypes

    import torch

    L = R.load()
    ref = torch.zeros((4, 100), dtype=torch.int32, device="cuda:0")
    gpu_ctx.set_reference(ref, 100, 4, 3)
    qs = torch.zeros((2, 4), dtype=torch.int32, device="cuda:0")
    out_i = torch.empty((2, 65), dtype=torch.int32, device="cuda:0")
    out_c = torch.empty((2, 65), dtype=torch.int16, device="cuda:0")
    rc = L.rfxp_topk(gpu_ctx.h, qs.data_ptr(), 4, 1, 2, None, 0, -1, 65, 0, out_i.data_ptr(), out_c.data_ptr())
    assert rc == 5  # K > 64 unsupported
    host = np.zeros(8, dtype=np.int32)
    rc = L.rfxp_topk(gpu_ctx.h, host.ctypes.data_as(ctypes.c_void_p), 4, 1, 2, None, 0, -1, 4, 0,
                     out_i.data_ptr(), out_c.data_ptr())
    assert rc == 1  # host pointer


def test_topk_scores_match_reference_formulas(gpu_ctx):
    """OOB queries: (float)count * (1.0f/|OOB(q)|) exactly as O.topk_oob;
    new queries: (float)count / (float)T."""
    import torch

    rng = np.random.default_rng(31)
    n, t, nleaf, k = 1200, 45, 7, 9
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    oob[:, 11] = 0
    gpu_ctx.set_reference(dev(leaf), n, t, nleaf)
    words = R.pack_oob_bits(dev(oob).to(torch.bool))
    idx, cnt = gpu_ctx.topk(dev(leaf), k, layout="tree", oob_words=words, exclude_base=0, positive_only=True)
    sc = gpu_ctx.topk_scores(idx, cnt, t, oob_words=words).cpu().numpy()
    for q in range(0, n, 7):
        wi, wc, ws = O.topk_oob(leaf, oob, q, k)
        m = len(wi)
        assert np.array_equal(sc[q, :m], ws) and (sc[q, m:] == 0).all(), q
    qs = rng.integers(0, nleaf, size=(50, t), dtype=np.int32)
    idx, cnt = gpu_ctx.topk(dev(qs), k)
    sc = gpu_ctx.topk_scores(idx, cnt, t).cpu().numpy()
    c = cnt.cpu().numpy().view(np.uint16).astype(np.float32)
    assert np.array_equal(sc, c / np.float32(t))


def test_pair_proximity_matches_oracle(gpu_ctx):
    import torch

    rng = np.random.default_rng(32)
    n, t, nleaf = 3000, 130, 9
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    leaf[rng.random((t, n)) < 0.05] = -1
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    oob[:, 17] = 0
    words = R.pack_oob_bits(dev(oob).to(torch.bool))
    pi = rng.integers(-2, n + 2, 700).astype(np.int64)
    pj = rng.integers(-2, n + 2, 700).astype(np.int64)
    pi[:5], pj[:5] = [17, 4, 9, 9, 0], [3, 4, 9, 17, n - 1]
    for layout in ("tree", "sample"):
        lf = leaf if layout == "tree" else np.ascontiguousarray(leaf.T)
        got = gpu_ctx.pair_proximity(dev(lf), words, n, t, nleaf, dev(pi), dev(pj), layout=layout).cpu().numpy()
        want = np.array([O.pair_proximity(leaf, oob, nleaf, a, b) for a, b in zip(pi, pj)], np.float32)
        assert np.array_equal(got, want), layout


@pytest.mark.parametrize("n,t,nleaf", [(2000, 100, 40), (70001, 12, 900)])
def test_outlier_full_mode_matches_oracle(gpu_ctx, n, t, nleaf):
    """Full mode: every training sample against the forest, itself excluded;
    raw within 1e-6 relative (float terms, double sums in different order),
    normalised scores by the host rule."""
    rng = np.random.default_rng(n + t)
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    gpu_ctx.set_reference(dev(leaf), n, t, nleaf)
    raw = gpu_ctx.outlier_raw(dev(leaf), layout="tree", exclude_base=0, numerator=float(n - 1),
                              isolated=float(n) * 1e10).cpu().numpy()
    sel = np.arange(n) if n <= 2000 else np.sort(rng.choice(n, 40, replace=False))
    want = O.outlier_raw(leaf, nleaf, np.ascontiguousarray(leaf[:, sel].T), exclude=sel.astype(np.int32),
                         numerator=float(n - 1), isolated=float(n) * 1e10)
    assert np.allclose(raw[sel], want, rtol=1e-6, atol=0)
    if n <= 2000:
        cls = (np.arange(n) % 3).astype(np.int32)
        for c in (None, cls):
            sc, _, _ = R.outlier_normalize(raw, c)
            assert np.allclose(sc, O.outlier_normalize(want, c), rtol=1e-5, atol=1e-5)


def test_outlier_anchor_mode_matches_oracle(gpu_ctx):
    rng = np.random.default_rng(33)
    n, t, nleaf = 5000, 60, 25
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    anchors = np.sort(rng.choice(n, 300, replace=False)).astype(np.int64)
    ex = np.full(n, -1, np.int32)
    ex[anchors] = np.arange(len(anchors))
    aleaf = np.ascontiguousarray(leaf[:, anchors])
    gpu_ctx.set_reference(dev(aleaf), len(anchors), t, nleaf)
    raw = gpu_ctx.outlier_raw(dev(leaf), layout="tree", exclude_idx=dev(ex), numerator=300.0,
                              isolated=300.0 * 1e10).cpu().numpy()
    want = O.outlier_raw(aleaf, nleaf, np.ascontiguousarray(leaf.T), exclude=ex, numerator=300.0,
                         isolated=300.0 * 1e10)
    assert np.allclose(raw, want, rtol=1e-6, atol=0)


def test_outlier_c5_scale_sampled_queries(gpu_ctx):
    """Full mode at the C5 reference size (N=1M, T=500, 2048 leaves) on a
    few training samples; the oracle costs N*T compares per query."""
    import torch

    n, t, nleaf = 1_000_000, 500, 2048
    g = torch.Generator(device="cuda:0")
    g.manual_seed(20261201 + 50)
    ref = torch.randint(0, nleaf, (t, n), generator=g, device="cuda:0", dtype=torch.int32)
    sel = np.array([0, 1, 500_000, 999_999], np.int64)
    gpu_ctx.set_reference(ref, n, t, nleaf)
    qs = ref[:, torch.from_numpy(sel).to("cuda:0")].T.contiguous()
    raw = gpu_ctx.outlier_raw(qs, exclude_idx=dev(sel.astype(np.int32)), numerator=float(n - 1),
                              isolated=float(n) * 1e10).cpu().numpy()
    want = O.outlier_raw(ref.cpu().numpy(), nleaf, qs.cpu().numpy(), exclude=sel.astype(np.int32),
                         numerator=float(n - 1), isolated=float(n) * 1e10)
    assert np.allclose(raw, want, rtol=1e-6, atol=0)
