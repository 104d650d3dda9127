"""rfxp_upper_noalloc (the allocation-free one-shot triangle) against the
rfxp_set_forest + rfxp_upper pair it combines: bit-exact, on two calls in a
row through the C ABI, the second with a smaller forest; plus its size limit
and argument checks.  The workspace it uses is static and shared, so the
second call also shows that nothing of the first call's index leaks."""
import numpy as np
import pytest

import rfxprox as R

pytestmark = pytest.mark.gpu


def forest(seed, n, t, nleaf, p_oob=0.368):
    rng = np.random.default_rng(seed)
    leaf = rng.integers(0, nleaf, size=(t, n)).astype(np.int32)
    oob = (rng.random((t, n)) < p_oob).astype(np.uint8)
    return leaf, oob


def device(leaf, oob):
    import torch

    lt = torch.from_numpy(leaf).to("cuda:0")
    ow = R.pack_oob_bits(torch.from_numpy(oob).to("cuda:0"))
    return lt, ow


def reference_rows(ctx, lt, ow, n, t, nleaf, fmt, r0, r1, scale, zp):
    """The existing entry points: rfxp_set_forest + rfxp_upper."""
    import torch

    ctx.set_forest(lt, ow, n, t, nleaf)
    out = torch.full((R.upper_nbytes(fmt, n, r0, r1) + 64,), 0x5A, dtype=torch.uint8, device="cuda:0")
    ctx.upper(fmt, out[:R.upper_nbytes(fmt, n, r0, r1)], r0, r1, scale=scale, zp=zp)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def noalloc_rows(ctx, lt, ow, n, t, nleaf, fmt, r0, r1, scale, zp):
    import torch

    out = torch.full((R.upper_nbytes(fmt, n, r0, r1) + 64,), 0x5A, dtype=torch.uint8, device="cuda:0")
    ctx.upper_noalloc(lt, ow, n, t, nleaf, fmt, out[:R.upper_nbytes(fmt, n, r0, r1)], r0, r1, scale=scale, zp=zp)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_set_forest_and_upper_on_two_calls(gpu_ctx):
    # call 1: a larger forest, uint8 codes of the whole triangle (T > 255:
    # the wrap check and the 16-bit recount path are live)
    cases = [
        (11, 3000, 300, 40, R.FMT_U8, 0, 3000, float(np.float32(1) / np.float32(255)), 0.0),
        # call 2: a smaller forest, fp32 entries of an unaligned row band
        (12, 1000, 40, 9, R.FMT_F32, 101, 977, 1.0, 0.0),
    ]
    for seed, n, t, nleaf, fmt, r0, r1, scale, zp in cases:
        assert R.upper_noalloc_workspace(n, t, nleaf) <= R.NOALLOC_MAX_BYTES
        leaf, oob = forest(seed, n, t, nleaf)
        lt, ow = device(leaf, oob)
        got = noalloc_rows(gpu_ctx, lt, ow, n, t, nleaf, fmt, r0, r1, scale, zp)
        want = reference_rows(gpu_ctx, lt, ow, n, t, nleaf, fmt, r0, r1, scale, zp)
        assert np.array_equal(got, want), f"N={n} T={t} fmt {fmt}: {int((got != want).sum())} bytes differ"
        assert (got[-64:] == 0x5A).all(), "write past the output"


def test_noalloc_with_a_caller_nout(gpu_ctx):
    """A device nout (with zeros, so 1/nout falls back to 1) given to the
    allocation-free call: the workspace then holds no OOB-count accumulator
    and 1/nout comes from the caller's counts.  Bit-exact against
    rfxp_set_forest(nout) + rfxp_upper, in fp32 (where 1/nout shows in every
    entry) and uint8 codes of an unaligned row band."""
    import torch

    n, t, nleaf = 1500, 300, 12
    leaf, oob = forest(31, n, t, nleaf)
    lt, ow = device(leaf, oob)
    nout = np.random.default_rng(32).integers(0, 5, size=n).astype(np.int32)
    nout[::7] = 0
    nt = torch.from_numpy(nout).to("cuda:0")
    assert R.upper_noalloc_workspace(n, t, nleaf, nout_given=True) <= R.NOALLOC_MAX_BYTES
    for fmt, r0, r1, scale in ((R.FMT_F32, 0, n, 1.0), (R.FMT_U8, 37, 1211, 1.0 / 4000.0)):
        nb = R.upper_nbytes(fmt, n, r0, r1)
        got = torch.full((nb + 64,), 0x5A, dtype=torch.uint8, device="cuda:0")
        gpu_ctx.upper_noalloc(lt, ow, n, t, nleaf, fmt, got[:nb], r0, r1, scale=scale, nout=nt)
        gpu_ctx.set_forest(lt, ow, n, t, nleaf, nout=nt)
        want = torch.full((nb + 64,), 0x5A, dtype=torch.uint8, device="cuda:0")
        gpu_ctx.upper(fmt, want[:nb], r0, r1, scale=scale)
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(g, w), f"fmt {fmt}: {int((g != w).sum())} bytes differ"
        assert (g[-64:] == 0x5A).all(), "write past the output"


def test_noalloc_leaves_the_context_forest_alone(gpu_ctx):
    import torch

    n, t, nleaf = 700, 30, 6
    leaf, oob = forest(21, n, t, nleaf)
    lt, ow = device(leaf, oob)
    gpu_ctx.set_forest(lt, ow, n, t, nleaf)
    before = torch.empty(R.upper_nbytes(R.FMT_U16, n), dtype=torch.uint8, device="cuda:0")
    gpu_ctx.upper(R.FMT_U16, before)
    leaf2, oob2 = forest(22, 500, 20, 4)
    lt2, ow2 = device(leaf2, oob2)
    noalloc_rows(gpu_ctx, lt2, ow2, 500, 20, 4, R.FMT_U8, 0, 500, 1.0 / 255.0, 0.0)
    after = torch.empty_like(before)
    gpu_ctx.upper(R.FMT_U16, after)
    torch.cuda.synchronize()
    assert torch.equal(before, after)


def test_noalloc_rejects_forests_beyond_the_workspace_and_bad_arguments(gpu_ctx):
    import torch

    n, t, nleaf = 20_000, 500, 4096     # C2 shape: ~330 MB of index
    assert R.upper_noalloc_workspace(n, t, nleaf) > R.NOALLOC_MAX_BYTES
    lt = torch.zeros((t, n), dtype=torch.int32, device="cuda:0")
    ow = torch.zeros((t, (n + 31) // 32), dtype=torch.int32, device="cuda:0")
    out = torch.empty(16, dtype=torch.uint8, device="cuda:0")
    with pytest.raises(R.RfxpError) as e:
        gpu_ctx.upper_noalloc(lt, ow, n, t, nleaf, R.FMT_U8, torch.empty(R.upper_nbytes(R.FMT_U8, n, 0, 1),
                                                                          dtype=torch.uint8, device="cuda:0"),
                              0, 1, scale=1.0 / 255.0)
    assert "workspace" in str(e.value)
    small = torch.zeros((4, 100), dtype=torch.int32, device="cuda:0")
    sw = torch.zeros((4, 4), dtype=torch.int32, device="cuda:0")
    with pytest.raises(R.RfxpError):  # scale 0 for a quantised format
        gpu_ctx.upper_noalloc(small, sw, 100, 4, 3, R.FMT_U8, torch.empty(R.upper_nbytes(R.FMT_U8, 100),
                                                                          dtype=torch.uint8, device="cuda:0"),
                              scale=0.0)
    raw = gpu_ctx._L.rfxp_upper_noalloc
    with pytest.raises(R.RfxpError):  # host output
        host = np.zeros(64, np.uint8)
        gpu_ctx._check(raw(gpu_ctx.h, small.data_ptr(), 1, 100, sw.data_ptr(), 4, 100, 4, 3, None, R.FMT_U8,
                           1.0, 0.0, 0, 1, host.ctypes.data))
    del out
