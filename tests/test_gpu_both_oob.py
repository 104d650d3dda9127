"""GPU parity of the both-OOB proximity (rfxp_both_oob) against the oracle's
brute force (orc_both_oob_rows, pinned in tests/test_oracle.py to an
independent numpy evaluation and a hand-worked case).  The reference has no
such mode, so parity is with that definition.  Bar: bit-exact counts and
bit-exact float quotients (one IEEE division of two exact integers)."""
import numpy as np
import pytest

import oracle as O
import rfxprox as R

pytestmark = pytest.mark.gpu


def dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def run(ctx, leaf, oob, nleaf, fmt, r0=0, r1=None, layout="tree"):
    import torch

    t, n = leaf.shape
    words = R.pack_oob_bits(dev(oob).to(torch.bool))
    lf = dev(leaf if layout == "tree" else np.ascontiguousarray(leaf.T))
    out = ctx.both_oob(lf, words, n, t, nleaf, fmt, r0, r1, layout=layout)
    got = out.cpu().numpy()
    return got.view(np.uint16) if fmt == R.FMT_U16 else got


@pytest.mark.parametrize("n,t,nleaf", [(1, 5, 2), (2, 31, 3), (63, 32, 4), (64, 33, 5), (65, 70, 3), (300, 40, 9)])
def test_both_oob_matches_oracle(gpu_ctx, n, t, nleaf):
    rng = np.random.default_rng(n + 100 * t)
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    leaf[rng.random((t, n)) < 0.05] = nleaf + 3      # invalid labels never match
    oob = (rng.random((t, n)) < 0.37).astype(np.uint8)
    if n > 1:
        oob[:, 0] = 0
    for fmt in (R.FMT_F32, R.FMT_U16):
        assert np.array_equal(run(gpu_ctx, leaf, oob, nleaf, fmt), O.both_oob_rows(leaf, oob, nleaf, fmt))


def test_both_oob_row_bands_and_sample_major(gpu_ctx):
    rng = np.random.default_rng(77)
    n, t, nleaf = 517, 90, 12
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.37).astype(np.uint8)
    for r0, r1 in [(0, 517), (5, 70), (64, 128), (200, 517), (516, 517), (10, 10)]:
        want = O.both_oob_rows(leaf, oob, nleaf, R.FMT_F32, r0, r1)
        assert np.array_equal(run(gpu_ctx, leaf, oob, nleaf, R.FMT_F32, r0, r1), want), (r0, r1)
    want = O.both_oob_rows(leaf, oob, nleaf, R.FMT_U16)
    assert np.array_equal(run(gpu_ctx, leaf, oob, nleaf, R.FMT_U16, layout="sample"), want)


def test_both_oob_c1_shape(gpu_ctx):
    """The benchmark configuration that names this normalisation: N = 2000,
    T = 100 (uniform synthetic leaves, Bernoulli(0.368) OOB)."""
    rng = np.random.default_rng(2000)
    n, t, nleaf = 2000, 100, 150
    leaf = rng.integers(0, nleaf, (t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    got = run(gpu_ctx, leaf, oob, nleaf, R.FMT_F32)
    assert np.array_equal(got, O.both_oob_rows(leaf, oob, nleaf, R.FMT_F32))
    assert (got >= 0).all() and (got <= 1).all()


def test_both_oob_rejects_bad_arguments(gpu_ctx):
    import torch

    leaf = torch.zeros((4, 10), dtype=torch.int32, device="cuda:0")
    words = torch.zeros((4, 1), dtype=torch.int32, device="cuda:0")
    with pytest.raises(R.RfxpError):
        gpu_ctx.both_oob(leaf, words, 10, 4, 3, R.FMT_U8)
    with pytest.raises(R.RfxpError):
        gpu_ctx.both_oob(leaf, words, 10, 4, 3, R.FMT_F32, 5, 3)
