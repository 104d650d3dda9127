"""GPU parity of the batched upper-triangle path (rfxp_set_forest + rfxp_upper)
against the CPU oracle, which is itself pinned to the compiled reference
(tests/test_oracle.py).  Bar: bit-exact for every format (counts, codes,
and the float formats, whose values are the same IEEE operations)."""
import numpy as np
import pytest

import oracle as O
import rfxprox as R
from closed_forms import pair_total, row_pair_counts
from tri_sums import symmetric_row_sums

pytestmark = pytest.mark.gpu


def make_forest(seed, n, t, nleaf, p_oob=0.368, p_invalid=0.0):
    rng = np.random.default_rng(seed)
    leaf = rng.integers(0, nleaf, size=(t, n), dtype=np.int64).astype(np.int32)
    if p_invalid > 0:
        bad = rng.random((t, n)) < p_invalid
        leaf[bad] = rng.choice(np.array([-1, nleaf, nleaf + 7, -5], dtype=np.int32), size=int(bad.sum()))
    oob = (rng.random((t, n)) < p_oob).astype(np.uint8)
    return leaf, oob


def upload(ctx, leaf, oob, nleaf, layout="tree", nout=None):
    import torch

    t, n = leaf.shape
    dev = torch.device("cuda:0")
    lt = torch.from_numpy(np.ascontiguousarray(leaf if layout == "tree" else leaf.T)).to(dev)
    ow = R.pack_oob_bits(torch.from_numpy(oob).to(dev))
    nt = None if nout is None else torch.from_numpy(np.ascontiguousarray(nout, dtype=np.int32)).to(dev)
    ctx.set_forest(lt, ow, n, t, nleaf, layout=layout, nout=nt)
    return lt, ow, nt


def gpu_rows(ctx, fmt, r0, r1, scale=1.0, zp=0.0, fill=0xA5, offset=0):
    """Runs rfxp_upper into a buffer pre-filled with `fill` and returns the
    bytes (as the oracle's dtype) plus the untouched guard bytes."""
    import torch

    nb = R.upper_nbytes(fmt, ctx.n, r0, r1)
    buf = torch.full((nb + 64 + offset,), fill, dtype=torch.uint8, device="cuda:0")
    view = buf[offset:offset + nb]
    ctx.upper(fmt, view, r0, r1, scale=scale, zp=zp)
    torch.cuda.synchronize()
    host = buf.cpu().numpy()
    out = host[offset:offset + nb]
    guard = np.concatenate([host[:offset], host[offset + nb:]])
    return out.view(O.FMT_DTYPE[fmt]), guard


def check_equal(got, want, what):
    if not np.array_equal(got, want):
        bad = np.nonzero(got != want)[0]
        raise AssertionError(f"{what}: {len(bad)} mismatches, first at {bad[:5]}: "
                             f"got {got[bad[:5]]} want {want[bad[:5]]}")


@pytest.mark.parametrize("n,t,nleaf", [(1, 1, 1), (2, 3, 2), (37, 5, 3), (300, 64, 17),
                                       (2000, 100, 64), (4099, 257, 300),
                                       (6000, 20, 5000),    # 2L > 8192: the whole-tree packing path
                                       (3000, 300, 5000)])  # whole-tree path with the byte-sum check
def test_counts_u16_match_oracle(gpu_ctx, n, t, nleaf):
    leaf, oob = make_forest(n * 31 + t, n, t, nleaf)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    got, guard = gpu_rows(gpu_ctx, O.FMT_U16, 0, n)
    want = O.upper_rows(leaf, oob, nleaf, O.FMT_U16)
    check_equal(got, want, f"U16 N={n} T={t}")
    assert (guard == 0xA5).all(), "write outside the output range"
    del keep


FMT_CASES = [
    (O.FMT_F32, 1.0, 0.0),
    (O.FMT_F16, 1.0, 0.0),
    (O.FMT_U16, 1.0, 0.0),
    (O.FMT_NF4, 1.0, 0.0),
    (O.FMT_U8, 1.0 / 255.0, -0.0),       # data-derived rule for min 0, max 1
    (O.FMT_U8, 1.0 / 4000.0, 3.0),       # codes depend on the column: exact path
    (O.FMT_U8, 1.0 / 60.0, 0.5),
    (O.FMT_I8, 1.0 / 127.0, 0.0),        # reference default int8 rule
    (O.FMT_I8, 1.0 / 2000.0, -100.0),
]


@pytest.mark.parametrize("fmt,scale,zp", FMT_CASES)
def test_formats_match_oracle(gpu_ctx, fmt, scale, zp):
    n, t, nleaf = 1531, 120, 23
    leaf, oob = make_forest(7, n, t, nleaf, p_invalid=0.02)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    got, guard = gpu_rows(gpu_ctx, fmt, 0, n, scale=np.float32(scale), zp=np.float32(zp))
    want = O.upper_rows(leaf, oob, nleaf, fmt, scale=np.float32(scale), zp=np.float32(zp))
    check_equal(got, want, f"fmt {fmt} scale {scale} zp {zp}")
    assert (guard == 0xA5).all()
    del keep


@pytest.mark.parametrize("fmt", [O.FMT_U8, O.FMT_NF4, O.FMT_F32, O.FMT_F16])
@pytest.mark.parametrize("r0,r1,offset", [(0, 1, 0), (3, 4, 1), (5, 400, 3), (101, 150, 0),
                                          (999, 1000, 2), (0, 1000, 5)])
def test_row_ranges(gpu_ctx, fmt, r0, r1, offset):
    n, t, nleaf = 1000, 50, 9
    leaf, oob = make_forest(11, n, t, nleaf)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    esz = {O.FMT_F32: 4, O.FMT_F16: 2}.get(fmt, 1)
    got, guard = gpu_rows(gpu_ctx, fmt, r0, r1, scale=np.float32(1 / 255.0), offset=offset * esz)
    want = O.upper_rows(leaf, oob, nleaf, fmt, scale=np.float32(1 / 255.0), r0=r0, r1=r1)
    if fmt == O.FMT_NF4:
        # boundary nibbles outside the range keep the buffer's fill value
        e0, e1 = O.tri_idx(n, r0, r0), O.tri_idx(n, r1, r1)
        want = want.copy()
        if e0 & 1:
            want[0] = (want[0] & 0xF0) | (0xA5 & 0x0F)
        if e1 & 1:
            want[-1] = (want[-1] & 0x0F) | (0xA5 & 0xF0)
    check_equal(got, want, f"fmt {fmt} rows {r0}:{r1}")
    assert (guard == 0xA5).all()
    del keep


@pytest.mark.parametrize("planted", [True, False])
def test_thousand_trees_check_with_per_thread_dummy_words(gpu_ctx, planted):
    """T = 1,000: four groups of 16 trees per wave, more counting steps than
    the shared dummy words allow, so the byte-sum check runs with one dummy
    word per thread (the path forests of 769 to 3,072 trees take).  Planted:
    samples 0..99 share sample 0's leaf in every tree, so their pairs reach
    counts near 465, which wrap 8 bits and must be recounted; otherwise
    counts stay near 2 and no item may be recounted."""
    n, t = 3000, 1000
    nleaf = 40 if planted else 200
    leaf, oob = make_forest(97 + planted, n, t, nleaf, p_oob=0.368)
    if planted:
        leaf[:, :100] = leaf[:, :1]
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    want_u = O.upper_rows(leaf, oob, nleaf, O.FMT_U16)
    assert (want_u.max() > 255) == planted
    for fmt, scale in ((O.FMT_U16, 1.0), (O.FMT_U8, 1 / 255.0)):
        scale = np.float32(scale)
        got, guard = gpu_rows(gpu_ctx, fmt, 0, n, scale=scale)
        want = want_u if fmt == O.FMT_U16 else O.upper_rows(leaf, oob, nleaf, fmt, scale=scale)
        check_equal(got, want, f"T=1000 planted={planted} fmt {fmt}")
        assert (guard == 0xA5).all()
        if planted:
            assert gpu_ctx.upper_recounts() > 0
        else:
            assert gpu_ctx.upper_recounts() == 0
    del keep


@pytest.mark.parametrize("case", ["every_pair_co_occurs", "entries_above_one", "zeros_and_diagonal"])
def test_data_derived_quantizer_scale(gpu_ctx, case):
    """rfxp_upper_minmax gives the min and max of the fp32 triangle, the
    data the reference's quantizer rule reads (compute_minmax over (float)P),
    for the whole triangle and for a row band; rfxp_quant_scale turns them
    into scale and zero point, under which the U8 and I8 codes equal the
    oracle's.  Cases: one leaf and T = 300, where every pair co-occurs
    (min > 0); caller nout of 0..2, which puts entries above 1 (max > 1);
    a sparse forest, where the rule gives the min 0 / max 1 parameters."""
    nout = None
    if case == "every_pair_co_occurs":
        n, t, nleaf = 400, 300, 1
        leaf, oob = make_forest(61, n, t, nleaf, p_oob=0.5)
    elif case == "entries_above_one":
        n, t, nleaf = 600, 40, 2
        leaf, oob = make_forest(62, n, t, nleaf)
        nout = np.random.default_rng(63).integers(0, 3, size=n).astype(np.int32)
    else:
        n, t, nleaf = 5000, 300, 2048
        leaf, oob = make_forest(64, n, t, nleaf)
    keep = upload(gpu_ctx, leaf, oob, nleaf, nout=nout)
    tri = O.upper_rows(leaf, oob, nleaf, O.FMT_F32, nout_arr=nout)
    mn, mx = gpu_ctx.upper_minmax()
    assert (mn, mx) == (float(tri.min()), float(tri.max()))
    r0 = n - 57
    band = tri[O.tri_idx(n, r0, r0):]
    assert gpu_ctx.upper_minmax(r0, n) == (float(band.min()), float(band.max()))
    if case == "every_pair_co_occurs":
        assert mn > 0
    elif case == "entries_above_one":
        assert mx > 1
    else:
        assert (mn, mx) == (0.0, 1.0)
    scale, zp = R.quant_scale(mn, mx)
    for fmt in (O.FMT_U8, O.FMT_I8):
        got, guard = gpu_rows(gpu_ctx, fmt, 0, n, scale=np.float32(scale), zp=np.float32(zp))
        want = O.upper_rows(leaf, oob, nleaf, fmt, scale=np.float32(scale), zp=np.float32(zp), nout_arr=nout)
        check_equal(got, want, f"{case} fmt {fmt} derived scale {scale} zp {zp}")
        assert (guard == 0xA5).all()
    del keep


def test_sample_major_layout_and_given_nout(gpu_ctx):
    n, t, nleaf = 777, 33, 5
    leaf, oob = make_forest(5, n, t, nleaf, p_invalid=0.05)
    nout = np.random.default_rng(3).integers(0, 4, size=n).astype(np.int32)  # includes zeros
    keep = upload(gpu_ctx, leaf, oob, nleaf, layout="sample", nout=nout)
    got, _ = gpu_rows(gpu_ctx, O.FMT_F32, 0, n)
    want = O.upper_rows(leaf, oob, nleaf, O.FMT_F32, nout_arr=nout)
    check_equal(got.view(np.uint32), want.view(np.uint32), "sample-major f32 with given nout")
    del keep


@pytest.mark.parametrize("fmt", [O.FMT_U16, O.FMT_U8, O.FMT_F32, O.FMT_NF4])
def test_counts_beyond_255_use_wide_counters(gpu_ctx, fmt):
    # one leaf and T=700: every pair co-occurs, U ~ Bin(700, 0.5) > 255
    n, t, nleaf = 300, 700, 1
    leaf, oob = make_forest(9, n, t, nleaf, p_oob=0.5)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    want_u = O.upper_rows(leaf, oob, nleaf, O.FMT_U16)
    assert want_u.max() > 255
    got, _ = gpu_rows(gpu_ctx, fmt, 0, n, scale=np.float32(1 / 255.0))
    want = O.upper_rows(leaf, oob, nleaf, fmt, scale=np.float32(1 / 255.0))
    check_equal(got, want, f"wide counters fmt {fmt}")
    assert gpu_ctx.upper_recounts() > 0   # the wrapped segments were recounted
    del keep


@pytest.mark.parametrize("fmt", [O.FMT_U16, O.FMT_U8, O.FMT_F32])
def test_many_trees_take_the_16bit_mode(gpu_ctx, fmt):
    """T = 3200: a wave's share of trees is more counting steps than the 8-bit
    byte-sum check covers, so every item is counted with 16-bit counters (the
    launch's 16-bit mode); few leaves make counts in the hundreds."""
    n, t, nleaf = 400, 3200, 3
    leaf, oob = make_forest(41, n, t, nleaf, p_oob=0.45, p_invalid=0.01)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    want_u = O.upper_rows(leaf, oob, nleaf, O.FMT_U16)
    assert want_u.max() > 600
    got, guard = gpu_rows(gpu_ctx, fmt, 0, n, scale=np.float32(1 / 255.0))
    check_equal(got, O.upper_rows(leaf, oob, nleaf, fmt, scale=np.float32(1 / 255.0)), f"16-bit mode fmt {fmt}")
    assert (guard == 0xA5).all()
    del keep


def test_split_rows_with_wrapped_8bit_counts(gpu_ctx):
    """N = 90,000 is above one workgroup's column segment, so rows below
    N - S are counted as two items.  T = 700 turns on the byte-sum check, and
    samples 0..299 share sample 0's leaf in every tree: their pairs reach
    counts near 325, which wrap 8 bits, inside both items of split rows.  Rows
    on both sides of the split boundary and of the group are compared, in
    every integer format: U8 with the min-0/max-1 rule, raw U16 counts, I8
    with a zero point, and U8 with codes that depend on the column (every
    nonzero count takes the exact per-column path)."""
    import torch

    n, t, nleaf = 90_000, 700, 400
    leaf, oob = make_forest(43, n, t, nleaf, p_oob=0.368)
    leaf[:, :300] = leaf[:, :1]
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    idx = O.RowIndex(leaf, oob, nleaf)
    assert idx.rows(O.FMT_U16, 0, 1)[:300].max() > 255
    # S = 81,472 columns per item on gfx950 (two workgroups' LDS per CU, dummy
    # words shared by the waves: T = 700 has at most 48 counting steps per wave)
    split = n - 81_472
    cases = [(O.FMT_U8, 1 / 255.0, 0.0), (O.FMT_U16, 1.0, 0.0), (O.FMT_I8, 1 / 2000.0, -100.0),
             (O.FMT_U8, 1 / 4000.0, 3.0)]
    for fmt, scale, zp in cases:
        scale, zp = np.float32(scale), np.float32(zp)
        out = torch.empty(R.upper_nbytes(fmt, n), dtype=torch.uint8, device="cuda:0")
        gpu_ctx.upper(fmt, out, 0, n, scale=scale, zp=zp)
        torch.cuda.synchronize()
        for r0 in (0, 1, 150, 298, 299, 300, split - 2, split, 40_000, n - 10):
            r1 = min(n, r0 + 3)
            want = idx.rows(fmt, r0, r1, scale, zp)
            e0, e1 = O.tri_idx(n, r0, r0), O.tri_idx(n, r1, r1)
            esz = np.dtype(O.FMT_DTYPE[fmt]).itemsize
            got = out[e0 * esz:e1 * esz].cpu().numpy().view(O.FMT_DTYPE[fmt])
            check_equal(got, want, f"fmt {fmt} scale {scale} zp {zp} rows {r0}:{r1}")
        del out
    assert gpu_ctx.upper_recounts() > 0
    idx.close()
    del keep


def test_all_oob_and_all_inbag_trees(gpu_ctx):
    n, t, nleaf = 500, 40, 4
    leaf, oob = make_forest(13, n, t, nleaf)
    oob[:10] = 1   # all OOB: no pairs
    oob[10:20] = 0  # all in-bag: no pairs
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    got, _ = gpu_rows(gpu_ctx, O.FMT_U16, 0, n)
    check_equal(got, O.upper_rows(leaf, oob, nleaf, O.FMT_U16), "degenerate trees")
    del keep


def test_deterministic(gpu_ctx):
    n, t, nleaf = 3000, 200, 50
    leaf, oob = make_forest(17, n, t, nleaf)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    a, _ = gpu_rows(gpu_ctx, O.FMT_U8, 0, n, scale=np.float32(1 / 255.0))
    b, _ = gpu_rows(gpu_ctx, O.FMT_U8, 0, n, scale=np.float32(1 / 255.0))
    assert np.array_equal(a, b)
    del keep


def test_rejects_bad_arguments(gpu_ctx):
    import torch

    n, t, nleaf = 100, 4, 3
    leaf, oob = make_forest(1, n, t, nleaf)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    out = torch.empty(R.upper_nbytes(O.FMT_U8, n), dtype=torch.uint8, device="cuda:0")
    with pytest.raises(R.RfxpError):
        gpu_ctx.upper(O.FMT_U8, out, 0, n, scale=0.0)
    raw = gpu_ctx._L.rfxp_upper
    with pytest.raises(R.RfxpError):
        gpu_ctx._check(raw(gpu_ctx.h, O.FMT_U8, 1.0, 0.0, 5, 3, out.data_ptr()))
    with pytest.raises(R.RfxpError):
        gpu_ctx._check(raw(gpu_ctx.h, 9, 1.0, 0.0, 0, n, out.data_ptr()))
    with pytest.raises(R.RfxpError):
        gpu_ctx._check(raw(gpu_ctx.h, O.FMT_U8, 1.0, float("nan"), 0, n, out.data_ptr()))
    host = np.zeros(16, dtype=np.uint8)
    with pytest.raises(R.RfxpError):
        gpu_ctx._check(gpu_ctx._L.rfxp_upper(gpu_ctx.h, O.FMT_U8, 1.0, 0.0, 0, 1, host.ctypes.data))
    del keep


def test_c1_forest_matches_reference_digests(gpu_ctx):
    """The first benchmark configuration's leaf matrix (CART forest, N=2000, T=100): the GPU
    triangle hashes to the digests of the reference's own cpu_proximity +
    cpu_finishprox output (tests/golden/make_golden.py)."""
    import hashlib
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "c1_forest.npz"))
    lab = g["label"].astype(np.int32)
    oob = (g["nin"] == 0).astype(np.uint8)
    nleaf = int(g["nleaf"])
    n = lab.shape[1]
    keep = upload(gpu_ctx, lab, oob, nleaf, nout=g["nout"])
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    u16, _ = gpu_rows(gpu_ctx, O.FMT_U16, 0, n)
    assert sha(u16) == str(g["sha_u16"])
    p32, _ = gpu_rows(gpu_ctx, O.FMT_F32, 0, n)
    assert sha(p32) == str(g["sha_p32"])
    u8, _ = gpu_rows(gpu_ctx, O.FMT_U8, 0, n, scale=np.float32(1) / np.float32(255))
    assert sha(u8) == str(g["sha_u8"])
    del keep


@pytest.mark.skip(reason="written for a 4-bit counter variant of the triangle kernel (one item per row); "
                         "that variant faulted the GPU at the C3 shape and is not in the library, and this "
                         "test has not run against the shipped 8-bit kernel")
@pytest.mark.parametrize("fmt,scale,zp", [(O.FMT_U8, 1.0 / 255.0, 0.0), (O.FMT_I8, 1.0 / 2000.0, -100.0)])
def test_rows_wider_than_a_segment_with_wrapping_counts(gpu_ctx, fmt, scale, zp):
    """N above the 8-bit segment width (rows split into two items).  A group
    of 300 samples shares every leaf, so its pairs reach U >= 16."""
    import torch

    n, t, nleaf = 80_000, 40, 400
    leaf, oob = make_forest(23, n, t, nleaf)
    leaf[:, :300] = leaf[:, :1]
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    out = torch.empty(R.upper_nbytes(fmt, n), dtype=torch.uint8, device="cuda:0")
    gpu_ctx.upper(fmt, out, 0, n, scale=np.float32(scale), zp=np.float32(zp))
    torch.cuda.synchronize()
    idx = O.RowIndex(leaf, oob, nleaf)
    u = idx.rows(O.FMT_U16, 0, 1)
    assert u[:300].max() >= 16
    for r0 in (0, 1, 150, 299, 300, 2_500, 40_000, 79_990):
        r1 = min(n, r0 + 10)
        want = idx.rows(fmt, r0, r1, np.float32(scale), np.float32(zp))
        e0, e1 = O.tri_idx(n, r0, r0), O.tri_idx(n, r1, r1)
        got = out[e0:e1].cpu().numpy().view(O.FMT_DTYPE[fmt])
        check_equal(got, want, f"fmt {fmt} rows {r0}:{r1}")
    idx.close()
    del keep


def test_c3_shape_sampled_rows(gpu_ctx):
    """Full north-star shape (N=100k, T=500, 2048 uniform leaves, uint8):
    rows spread over the triangle equal the oracle's; all codes are in the
    range the normalisation allows."""
    import torch

    n, t, nleaf = 100_000, 500, 2048
    g = torch.Generator(device="cuda:0")
    g.manual_seed(20261204)
    leaf = torch.randint(0, nleaf, (t, n), generator=g, device="cuda:0", dtype=torch.int32)
    oob = torch.rand((t, n), generator=g, device="cuda:0") < 0.368
    words = R.pack_oob_bits(oob)
    gpu_ctx.set_forest(leaf, words, n, t, nleaf)
    scale = float(np.float32(1) / np.float32(255))
    out = torch.empty(R.upper_nbytes(O.FMT_U8, n), dtype=torch.uint8, device="cuda:0")
    gpu_ctx.upper(O.FMT_U8, out, 0, n, scale=scale, zp=0.0)
    torch.cuda.synchronize()
    leaf_np = leaf.cpu().numpy()
    oob_np = oob.to(torch.uint8).cpu().numpy()
    idx = O.RowIndex(leaf_np, oob_np, nleaf)
    for r0 in (0, 1, 777, 31_313, 50_000, 77_777, 99_990):
        r1 = min(n, r0 + 10)
        want = idx.rows(O.FMT_U8, r0, r1, scale, 0.0)
        e0, e1 = O.tri_idx(n, r0, r0), O.tri_idx(n, r1, r1)
        got = out[e0:e1].cpu().numpy()
        check_equal(got, want, f"C3 rows {r0}:{r1}")
    # diagonal entries are code(1.0): the reference quantizer truncates
    # 1/fl(1/255) = 254.99998 to 254
    dcode = O.q_u8(1.0, scale, 0.0)
    assert dcode == 254
    diag = torch.tensor([O.tri_idx(n, i, i) for i in range(0, n, 997)], device="cuda:0")
    assert bool((out[diag] == dcode).all())
    idx.close()


@pytest.mark.parametrize("n,t,nleaf", [
    (100_000, 500, 2048),   # C3: per-part packing, sorted member scatter
    (100_000, 200, 25_000),  # whole-tree packing: range histograms, offsets read from L2
])
def test_whole_triangle_invariants(gpu_ctx, n, t, nleaf):
    """Raw U16 counts over the whole triangle (5e9 entries at N = 100k):
    their sum equals the closed form from the leaf histograms (pair_total),
    every sample's sum over its row and column equals the sizes of its
    opposite buckets summed over the trees (row_pair_counts; a count in the
    wrong column of the right row keeps the total but not these), every
    count lies in [0, T], and the diagonal is 0."""
    import torch

    g = torch.Generator(device="cuda:0")
    g.manual_seed(20261205 + nleaf)
    leaf = torch.randint(0, nleaf, (t, n), generator=g, device="cuda:0", dtype=torch.int32)
    oob = torch.rand((t, n), generator=g, device="cuda:0") < 0.368
    words = R.pack_oob_bits(oob)
    gpu_ctx.set_forest(leaf, words, n, t, nleaf)
    out = torch.empty(R.upper_nbytes(O.FMT_U16, n), dtype=torch.uint8, device="cuda:0")
    gpu_ctx.upper(O.FMT_U16, out, 0, n)
    torch.cuda.synchronize()
    u = out.view(torch.int16)  # counts <= 500 read the same as int16
    leaf_np, oob_np = leaf.cpu().numpy(), oob.to(torch.uint8).cpu().numpy()
    got_total = int(u.sum(dtype=torch.int64).item())
    want_total = pair_total(leaf_np, oob_np, nleaf)
    assert got_total == want_total, (got_total, want_total)
    got_rows = symmetric_row_sums(u, n).cpu().numpy()
    want_rows = row_pair_counts(leaf_np, oob_np, nleaf)
    bad = np.nonzero(got_rows != want_rows)[0]
    assert bad.size == 0, (bad.size, bad[:5], got_rows[bad[:5]], want_rows[bad[:5]])
    assert int(u.max().item()) <= t and int(u.min().item()) >= 0
    diag = torch.tensor([O.tri_idx(n, i, i) for i in range(0, n, 613)], device="cuda:0")
    assert bool((u[diag] == 0).all())
    del out, u


def test_c2_shape_full_triangle_f32(gpu_ctx):
    """The second benchmark configuration's shape: N=20,000, T=500, 1,000-4,096 leaves per tree
    (the per-part packing path), fp32 output.  The whole triangle (2e8
    entries) equals the oracle's bit for bit, and so do the raw counts."""
    import torch

    n, t = 20_000, 500
    rng = np.random.default_rng(20261203)
    lt = rng.integers(1000, 4097, size=t)
    leaf = (rng.random((t, n)) * lt[:, None]).astype(np.int32)
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    nleaf = 4096
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    idx = O.RowIndex(leaf, oob, nleaf)
    for fmt in (O.FMT_F32, O.FMT_U16):
        out = torch.empty(R.upper_nbytes(fmt, n), dtype=torch.uint8, device="cuda:0")
        gpu_ctx.upper(fmt, out, 0, n)
        torch.cuda.synchronize()
        # T > 255 runs the byte-sum wrap check; counts here stay far below 256,
        # so no row segment may be recounted (a spurious recount rewrites it)
        assert gpu_ctx.upper_recounts() == 0, fmt
        got = out.cpu().numpy().view(O.FMT_DTYPE[fmt])
        want = idx.rows(fmt, 0, n)
        if fmt == O.FMT_F32:
            check_equal(got.view(np.uint32), want.view(np.uint32), "C2 f32 triangle")
        else:
            check_equal(got, want, "C2 u16 triangle")
            assert int(want.max()) <= t
        del out
    idx.close()
    del keep


def test_c2_data_grown_regression_forest(gpu_ctx):
    """The second benchmark configuration's data (N = 20,000, p = 50, y = sin(x0) + x1 x2 +
    N(0, 0.1)) through a forest grown on it (sklearn CART, mtry 17, leaves of
    at least 5 samples, seeded bootstrap; 100 of the config's 500 trees to
    keep the growing short): ~2,000 leaves per tree of skewed sizes, labels
    that are node ids (so most label values are internal nodes, never used),
    OOB bits from each tree's bootstrap sample.  The whole fp32 triangle and
    the raw counts equal the oracle's bit for bit."""
    import torch

    ens = pytest.importorskip("sklearn.ensemble")
    rng = np.random.default_rng(20261201 + 2)
    n, p, t = 20_000, 50, 100
    X = rng.standard_normal((n, p)).astype(np.float32)
    y = np.sin(X[:, 0]) + X[:, 1] * X[:, 2] + rng.normal(0.0, 0.1, n)
    rf = ens.RandomForestRegressor(n_estimators=t, max_features=17, min_samples_leaf=5, bootstrap=True,
                                   n_jobs=8, random_state=5).fit(X, y)
    leaf = np.ascontiguousarray(rf.apply(X).T.astype(np.int32))    # (T, N) node ids
    oob = np.ones((t, n), dtype=np.uint8)
    for k, idx in enumerate(rf.estimators_samples_):
        oob[k, idx] = 0
    nleaf = int(leaf.max()) + 1
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    ridx = O.RowIndex(leaf, oob, nleaf)
    for fmt in (O.FMT_F32, O.FMT_U16):
        out = torch.empty(R.upper_nbytes(fmt, n), dtype=torch.uint8, device="cuda:0")
        gpu_ctx.upper(fmt, out, 0, n)
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(O.FMT_DTYPE[fmt])
        want = ridx.rows(fmt, 0, n)
        if fmt == O.FMT_F32:
            check_equal(got.view(np.uint32), want.view(np.uint32), "grown C2 forest f32 triangle")
        else:
            check_equal(got, want, "grown C2 forest u16 triangle")
        del out
    ridx.close()
    del keep


@pytest.mark.parametrize("case", ["parts", "whole_tree"])
def test_buckets_beyond_16383_members(gpu_ctx, case):
    """Buckets of 16,383 or more members take the read-to-the-mark path of
    the hit phase.  'parts': two leaves at N=60,000 (per-part packing);
    'whole_tree': 2L > 8192 with one leaf holding 40,000 samples (whole-tree
    packing)."""
    import torch

    n = 60_000
    rng = np.random.default_rng(31 if case == "parts" else 37)
    if case == "parts":
        t, nleaf = 20, 2
        leaf = rng.integers(0, nleaf, size=(t, n)).astype(np.int32)
    else:
        t, nleaf = 12, 5000
        leaf = rng.integers(1, nleaf, size=(t, n)).astype(np.int32)
        big = rng.random((t, n)) < 40_000 / n
        leaf[big] = 0
    oob = (rng.random((t, n)) < 0.368).astype(np.uint8)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    idx = O.RowIndex(leaf, oob, nleaf)
    for fmt, scale in ((O.FMT_U16, 1.0), (O.FMT_U8, float(np.float32(1) / np.float32(255)))):
        out = torch.empty(R.upper_nbytes(fmt, n), dtype=torch.uint8, device="cuda:0")
        gpu_ctx.upper(fmt, out, 0, n, scale=scale)
        torch.cuda.synchronize()
        esz = 2 if fmt == O.FMT_U16 else 1
        for r0 in (0, 1, 4_999, 16_383, 30_000, 59_990):
            r1 = min(n, r0 + 10)
            e0, e1 = O.tri_idx(n, r0, r0), O.tri_idx(n, r1, r1)
            got = out[e0 * esz:e1 * esz].cpu().numpy().view(O.FMT_DTYPE[fmt])
            check_equal(got, idx.rows(fmt, r0, r1, scale, 0.0), f"{case} fmt {fmt} rows {r0}:{r1}")
        del out
    idx.close()
    del keep


@pytest.mark.parametrize("n,t,nleaf,plan", [
    (600_000, 3, 16, R.PACK_PARTS_DIRECT),      # parts of 75,000 > 65,535 samples
    (200_000, 6, 256, R.PACK_PARTS_SORTED2),    # 2-byte staging keeps two workgroups per CU
    (50_000, 6, 64, R.PACK_PARTS_SORTED4),       # keys of a part held in registers
    (200_000, 4, 2048, R.PACK_PARTS_SORTED4),    # parts of 25,000: keys read twice
    (140_000, 6, 4096, R.PACK_PARTS_SORTED4),   # 8,192 buckets, one workgroup per CU
])
def test_member_scatter_variants(gpu_ctx, n, t, nleaf, plan):
    """Each member-scatter kernel of the per-part packing path (the plan
    query names the one this shape takes) gives the oracle's counts: row bands
    at the start, middle and end of the triangle, raw U16 counts, 2% invalid
    labels."""
    assert R.pack_plan(n, t, nleaf) == plan
    leaf, oob = make_forest(n + nleaf, n, t, nleaf, p_invalid=0.02)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    idx = O.RowIndex(leaf, oob, nleaf)
    for r0 in (0, n // 2 - 1, n - 3):
        r1 = r0 + 3
        got, guard = gpu_rows(gpu_ctx, O.FMT_U16, r0, r1)
        check_equal(got, idx.rows(O.FMT_U16, r0, r1, 1.0, 0.0), f"plan {plan} rows {r0}:{r1}")
        assert (guard == 0xA5).all()
    idx.close()
    del keep


def test_row_bands_back_to_back_on_the_context_stream():
    """Two row bands queued on the context's own (non-blocking) stream with
    no synchronisation between them, the second band no larger than the
    first: each equals the oracle, and nothing is written outside either
    buffer."""
    import torch

    n, t, nleaf = 3000, 60, 40
    leaf, oob = make_forest(41, n, t, nleaf)
    ctx = R.Context(0)  # own stream
    lt = torch.from_numpy(leaf).to("cuda:0")
    ow = R.pack_oob_bits(torch.from_numpy(oob).to("cuda:0"))
    torch.cuda.synchronize()
    ctx.set_forest(lt, ow, n, t, nleaf)
    bands = [(0, 1800), (1800, 3000), (100, 900)]
    bufs = []
    for r0, r1 in bands:
        nb = R.upper_nbytes(O.FMT_U16, n, r0, r1)
        bufs.append(torch.full((nb + 64,), 0xA5, dtype=torch.uint8, device="cuda:0"))
    torch.cuda.synchronize()
    for (r0, r1), b in zip(bands, bufs):
        ctx.upper(O.FMT_U16, b[:R.upper_nbytes(O.FMT_U16, n, r0, r1)], r0, r1)
    ctx.sync()
    for (r0, r1), b in zip(bands, bufs):
        host = b.cpu().numpy()
        nb = R.upper_nbytes(O.FMT_U16, n, r0, r1)
        check_equal(host[:nb].view(np.uint16), O.upper_rows(leaf, oob, nleaf, O.FMT_U16, r0=r0, r1=r1),
                    f"band {r0}:{r1}")
        assert (host[nb:] == 0xA5).all()
    ctx.close()


def test_per_part_back_to_back_placement_past_the_line_fit_bound(gpu_ctx):
    """N = 33,000 with 1,031 leaves takes the per-part packing path; with
    10,640 trees the line-fit layout would need T x 100,928 ids, past 2^30,
    so the buckets are placed back to back (tree stride N) instead, and
    10,640 trees count in the 16-bit mode.  Sampled rows at both ends and in
    the middle, U16 and U8, against the oracle."""
    n, t, nleaf = 33_000, 10_640, 1031
    nb = 2 * nleaf
    assert n >= 32_768 and n >= 16 * nb                       # per-part path
    stride = (n + 31 * (nb + (nb + 15) // 16) + 31) // 32 * 32
    assert t * stride + 64 >= 1 << 30 and n * t + 64 < (1 << 30) - 1
    leaf, oob = make_forest(77, n, t, nleaf, p_oob=0.368)
    keep = upload(gpu_ctx, leaf, oob, nleaf)
    idx = O.RowIndex(leaf, oob, nleaf)
    for fmt, scale, r0, r1 in [(O.FMT_U16, 1.0, 0, 3), (O.FMT_U8, 1 / 255.0, 16_500, 16_503),
                               (O.FMT_U16, 1.0, n - 3, n)]:
        got, guard = gpu_rows(gpu_ctx, fmt, r0, r1, scale=np.float32(scale))
        check_equal(got, idx.rows(fmt, r0, r1, np.float32(scale), np.float32(0.0)), f"fmt {fmt} rows {r0}:{r1}")
        assert (guard == 0xA5).all()
    idx.close()
    del keep
