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


def test_invalid_labels_never_match(gpu_ctx):
    rng = np.random.default_rng(5)
    n, t, nleaf, q, k = 3000, 20, 11, 10, 30
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    ref[rng.random((t, n)) < 0.1] = -1
    qs = rng.integers(0, nleaf, size=(q, t), dtype=np.int32)
    qs[rng.random((q, t)) < 0.2] = -2
    got_i, got_c = run_topk(gpu_ctx, ref, nleaf, qs, k)
    want_i, want_c = O.topk_all(ref, qs, k)
    assert np.array_equal(got_c, want_c) and np.array_equal(got_i, want_i)


def test_exclude_self(gpu_ctx):
    rng = np.random.default_rng(8)
    n, t, nleaf, k = 900, 30, 6, 12
    ref = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    qs = np.ascontiguousarray(ref[:, 100:140].T)   # training samples 100..139 as queries
    got_i, got_c = run_topk(gpu_ctx, ref, nleaf, qs, k, exclude_base=100)
    want_i, want_c = O.topk_all(ref, qs, k, exclude=np.arange(100, 140, dtype=np.int32))
    assert np.array_equal(got_c, want_c) and np.array_equal(got_i, want_i)


def test_oob_query_semantics(gpu_ctx):
    import torch

    rng = np.random.default_rng(13)
    n, t, nleaf, k = 1500, 60, 8, 10
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    oob[:, 7] = 0                                    # a sample never OOB: no results
    gpu_ctx.set_reference(dev(leaf), n, t, nleaf)
    words = R.pack_oob_bits(dev(oob).to(torch.bool))
    idx, cnt = gpu_ctx.topk(dev(leaf), k, layout="tree", oob_words=words, exclude_base=0,
                            positive_only=True)
    idx, cnt = idx.cpu().numpy(), cnt.cpu().numpy().view(np.uint16)
    for q in range(n):
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
