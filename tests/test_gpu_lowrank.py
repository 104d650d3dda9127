"""GPU low-rank path (rfxp_lowrank_pv, rfxp_lowrank_subspace) against the
oracle's double-precision one-hot SpMM (pinned in tests/test_oracle.py to the
dense product A A^T V / T) and a numpy subspace iteration in double.
Tolerances: P V within 1e-5 relative Frobenius (fp32 sums of at most T*N
terms); Q B Q^T V within 1e-4 relative Frobenius, as the north star states."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def zipf_leaves(rng, n, t, nleaf, s=1.1):
    p = 1.0 / np.arange(1, nleaf + 1) ** s
    p /= p.sum()
    leaf = np.empty((t, n), dtype=np.int32)
    for k in range(t):
        perm = rng.permutation(nleaf).astype(np.int32)
        leaf[k] = perm[rng.choice(nleaf, size=n, p=p)]
    return leaf


def dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def rel_fro(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("n,t,nleaf,r", [(1, 1, 1, 1), (300, 7, 5, 3), (5000, 20, 40, 32),
                                         (20000, 12, 64, 17), (9000, 9, 3, 64)])
def test_pv_matches_oracle(gpu_ctx, n, t, nleaf, r):
    rng = np.random.default_rng(n + r)
    leaf = zipf_leaves(rng, n, t, nleaf)   # skewed: the big leaves span several pieces
    if n > 100:
        leaf[rng.random((t, n)) < 0.03] = -1
    V = rng.standard_normal((n, r)).astype(np.float32)
    lt = dev(leaf)
    gpu_ctx.set_reference(lt, n, t, nleaf)
    Y = gpu_ctx.lowrank_pv(dev(V)).cpu().numpy()
    want = O.lowrank_pv(leaf, nleaf, V.astype(np.float64))
    assert rel_fro(Y.astype(np.float64), want) < 1e-5


def test_pv_repeat_runs_differ_only_by_rounding(gpu_ctx):
    """k_lr_w adds the partial sums of a leaf split over several pieces with
    float atomics, whose order varies between runs: P V is not bit-for-bit
    repeatable for such forests, but repeated runs agree to fp32 rounding
    (1e-6 relative Frobenius, far inside the 1e-5 contract) and each stays
    within that contract of the double-precision oracle.  The leaf matrix is
    handed over as a temporary: the binding keeps it alive for the later
    P V calls (rfxp_lowrank_pv reads it), even when V takes a block of the
    same size."""
    rng = np.random.default_rng(77)
    n, t, nleaf, r = 60_000, 16, 6, 16   # Zipf(1.1) over 6 leaves: leaves of ~25,000 members split
    leaf = zipf_leaves(rng, n, t, nleaf)
    V = rng.standard_normal((n, r)).astype(np.float32)
    gpu_ctx.set_reference(dev(leaf), n, t, nleaf)
    runs = [gpu_ctx.lowrank_pv(dev(V)).cpu().numpy().astype(np.float64) for _ in range(4)]
    want = O.lowrank_pv(leaf, nleaf, V.astype(np.float64))
    for Y in runs:
        assert rel_fro(Y, want) < 1e-5
        assert rel_fro(Y, runs[0]) < 1e-6


def numpy_subspace(leaf, nleaf, V0, iters):
    def orth(X):
        Q, R = np.linalg.qr(X)
        return Q * np.sign(np.diag(R))

    Q = orth(V0.astype(np.float64))
    for _ in range(iters):
        Q = orth(O.lowrank_pv(leaf, nleaf, Q))
    B = Q.T @ O.lowrank_pv(leaf, nleaf, Q)
    return Q, B


def test_subspace_matches_numpy(gpu_ctx):
    rng = np.random.default_rng(4)
    n, t, nleaf, r, iters = 6000, 30, 24, 8, 5
    leaf = zipf_leaves(rng, n, t, nleaf)
    V0 = rng.standard_normal((n, r)).astype(np.float32)
    lt = dev(leaf)
    gpu_ctx.set_reference(lt, n, t, nleaf)
    Q, B = gpu_ctx.lowrank_subspace(dev(V0), iters)
    Q = Q.cpu().numpy().astype(np.float64)
    Qw, Bw = numpy_subspace(leaf, nleaf, V0, iters)
    assert np.abs(Q.T @ Q - np.eye(r)).max() < 1e-5
    Vt = rng.standard_normal((n, r))
    assert rel_fro(Q @ (B @ (Q.T @ Vt)), Qw @ (Bw @ (Qw.T @ Vt))) < 1e-4


def test_rank32_subspace_at_100k_matches_numpy(gpu_ctx):
    """The rank-32, 5-iteration factor at N = 100,000 against numpy's
    subspace iteration in double (same start block), within the 1e-4
    relative Frobenius contract on Q B Q^T applied to a random block."""
    rng = np.random.default_rng(8)
    n, t, nleaf, r, iters = 100_000, 40, 48, 32, 5
    leaf = zipf_leaves(rng, n, t, nleaf)
    V0 = rng.standard_normal((n, r)).astype(np.float32)
    gpu_ctx.set_reference(dev(leaf), n, t, nleaf)
    Q, B = gpu_ctx.lowrank_subspace(dev(V0), iters)
    Q = Q.cpu().numpy().astype(np.float64)
    Qw, Bw = numpy_subspace(leaf, nleaf, V0, iters)
    assert np.abs(Q.T @ Q - np.eye(r)).max() < 1e-5
    Vt = rng.standard_normal((n, r))
    assert rel_fro(Q @ (B @ (Q.T @ Vt)), Qw @ (Bw @ (Qw.T @ Vt))) < 1e-4


def test_c4_shape_properties(gpu_ctx):
    """Config C4 shape (N=1M, T=500, 4096 leaves, Zipf(1.1) sizes, a label
    permutation per tree) through properties the size does not change:
    P 1 = (1/T) sum_t |leaf_i(t)| exactly (in fp32 rounding), P is
    symmetric (u . P v = v . P u), and P V on sampled rows equals an
    independent double evaluation within the 1e-5 contract."""
    import torch

    n, t, nleaf = 1_000_000, 500, 4096
    g = torch.Generator(device="cuda:0")
    g.manual_seed(20261201 + 4)
    p = 1.0 / torch.arange(1, nleaf + 1, dtype=torch.float64) ** 1.1
    p = (p / p.sum()).to("cuda:0")
    leaf = torch.empty((t, n), dtype=torch.int32, device="cuda:0")
    for k in range(t):
        perm = torch.randperm(nleaf, generator=g, device="cuda:0").to(torch.int32)
        leaf[k] = perm[torch.multinomial(p, n, replacement=True, generator=g)]
    gpu_ctx.set_reference(leaf, n, t, nleaf)
    ones = torch.ones((n, 8), dtype=torch.float32, device="cuda:0")
    Y = gpu_ctx.lowrank_pv(ones)
    sizes = torch.zeros((t, nleaf), dtype=torch.float64, device="cuda:0")
    sizes.scatter_add_(1, leaf.long(), torch.ones((t, n), dtype=torch.float64, device="cuda:0"))
    want = torch.gather(sizes, 1, leaf.long()).sum(0) / t
    err = ((Y[:, 0].double() - want).abs() / want).max().item()
    assert err < 1e-5
    assert (Y == Y[:, :1]).all()
    u = torch.randn((n, 4), generator=g, device="cuda:0")
    v = torch.randn((n, 4), generator=g, device="cuda:0")
    Pu, Pv = gpu_ctx.lowrank_pv(u), gpu_ctx.lowrank_pv(v)
    a = (u.double() * Pv.double()).sum(0)
    b = (v.double() * Pu.double()).sum(0)
    scale = u.double().norm(dim=0) * Pv.double().norm(dim=0)
    assert ((a - b).abs() / scale).max().item() < 1e-5
    # P V itself on 128 sampled rows against an exact double evaluation that
    # shares nothing with the library's kernels: per tree, the double sums of
    # V over the leaves the sampled rows sit in (torch index_add), averaged
    # over the trees
    r = 32
    V = torch.randn((n, r), generator=g, device="cuda:0")
    Y = gpu_ctx.lowrank_pv(V)
    rows = torch.randint(0, n, (128,), generator=g, device="cuda:0")
    V64 = V.double()
    want = torch.zeros((rows.numel(), r), dtype=torch.float64, device="cuda:0")
    slot_of = torch.full((nleaf,), -1, dtype=torch.int64, device="cuda:0")
    for k in range(t):
        lk = leaf[k].long()
        labels, inv = torch.unique(lk[rows], return_inverse=True)
        slot_of[labels] = torch.arange(labels.numel(), device="cuda:0")
        slot = slot_of[lk]
        sel = torch.nonzero(slot >= 0).squeeze(1)
        W = torch.zeros((labels.numel(), r), dtype=torch.float64, device="cuda:0")
        W.index_add_(0, slot[sel], V64[sel])
        want += W[inv]
        slot_of[labels] = -1
    want /= t
    got = Y[rows].double()
    assert ((got - want).norm() / want.norm()).item() < 1e-5


@pytest.mark.parametrize("n,t,nleaf,r,layout", [(1, 2, 1, 1, "tree"), (1500, 40, 12, 8, "tree"),
                                                (4000, 25, 30, 32, "sample")])
def test_oob_normalised_pv_matches_finishprox_matrix(gpu_ctx, n, t, nleaf, r, layout):
    """Y = P V for the cpu_finishprox matrix P of the forest's OOB counts:
    the dense P here rounds to the oracle's F32 triangle (pinned to the
    compiled reference), and the SpMM matches P V within 1e-6."""
    import torch

    import rfxprox as R

    rng = np.random.default_rng(n + t + r)
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    leaf[rng.random((t, n)) < 0.03] = -1
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    if n > 1:
        oob[:, 1] = 0   # never OOB: r = 1
    words = R.pack_oob_bits(dev(oob).to(torch.bool))
    lf = dev(leaf if layout == "tree" else np.ascontiguousarray(leaf.T))  # kept alive: the SpMM reads it
    gpu_ctx.set_forest(lf, words, n, t, nleaf, layout=layout)
    U = np.zeros((n, n))
    U[np.triu_indices(n)] = O.upper_counts_scatter(leaf, oob, nleaf)
    U = U + np.triu(U, 1).T
    nout = oob.sum(axis=0)
    rv = np.where(nout > 0, 1.0 / np.maximum(nout, 1), 1.0)
    P = 0.25 * (rv[:, None] * U + U * rv[None, :]) + np.eye(n)
    assert np.array_equal(P[np.triu_indices(n)].astype(np.float32), O.upper_rows(leaf, oob, nleaf, O.FMT_F32))
    V = rng.standard_normal((n, r)).astype(np.float32)
    Y = gpu_ctx.lowrank_oob_pv(dev(V)).cpu().numpy()
    assert rel_fro(Y.astype(np.float64), P @ V.astype(np.float64)) <= 1e-6


def test_oob_normalised_pv_with_temporary_forest_inputs(gpu_ctx):
    """The forest's leaf matrix and OOB words handed over as temporaries: the
    binding keeps them alive for rfxp_lowrank_oob_pv, which reads them after
    rfxp_set_forest returns, even when V takes a freed block of the same size
    (leaf: 8 x 4000 int32; V: 4000 x 8 float32)."""
    import torch

    import rfxprox as R

    rng = np.random.default_rng(5)
    n, t, nleaf, r = 4000, 8, 9, 8
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int32)
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    gpu_ctx.set_forest(dev(leaf), R.pack_oob_bits(dev(oob).to(torch.bool)), n, t, nleaf)
    U = np.zeros((n, n))
    U[np.triu_indices(n)] = O.upper_counts_scatter(leaf, oob, nleaf)
    U = U + np.triu(U, 1).T
    nout = oob.sum(axis=0)
    rv = np.where(nout > 0, 1.0 / np.maximum(nout, 1), 1.0)
    P = 0.25 * (rv[:, None] * U + U * rv[None, :]) + np.eye(n)
    V = rng.standard_normal((n, r)).astype(np.float32)
    Y = gpu_ctx.lowrank_oob_pv(dev(V)).cpu().numpy()
    assert rel_fro(Y.astype(np.float64), P @ V.astype(np.float64)) <= 1e-6
