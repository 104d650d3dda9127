"""The library's own HIP kernels run on the CPU by the emulator in tests/emu
(every GPU thread a coroutine, wave builtins resolved per 64-lane wave over
the lanes that reach them, device memory and each workgroup's LDS from
malloc, AddressSanitizer on),
through the C ABI, against the oracle.  These runs check index arithmetic,
buffer sizes and bounds on every packing path and format without a GPU: an
access outside an allocation or outside a workgroup's LDS aborts the run
with the sanitizer's report.  They do not replace the GPU parity tests; the
emulation knows nothing of timing, occupancy or the hardware's memory
model."""
import os
import struct
import subprocess

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
EMU = os.path.join(HERE, "emu")


@pytest.fixture(scope="module")
def driver(emu_driver):
    return emu_driver


def pack_words(oob):
    t, n = oob.shape
    w = (n + 31) // 32
    pad = np.zeros((t, w * 32), np.uint64)
    pad[:, :n] = oob
    return (pad.reshape(t, w, 32) << np.arange(32, dtype=np.uint64)).sum(axis=2).astype(np.uint32)


def emulate(driver, tmp_path, mode, leaf, oob, nleaf, fmt=O.FMT_U16, scale=1.0, zp=0.0, r0=0, r1=None,
            nout=None, layout="tree", V=None, env_extra=None):
    t, n = leaf.shape
    r1 = n if r1 is None else r1
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(struct.pack("<iqiiiffqqii", mode, n, t, nleaf, fmt, np.float32(scale), np.float32(zp), r0, r1,
                            int(nout is not None), int(layout == "sample")))
        np.ascontiguousarray(leaf if layout == "tree" else leaf.T, dtype=np.int32).tofile(f)
        pack_words(oob).tofile(f)
        if nout is not None:
            np.asarray(nout, np.int32).tofile(f)
        if V is not None:
            np.ascontiguousarray(V, np.float32).tofile(f)
    env = dict(os.environ, ASAN_OPTIONS="detect_stack_use_after_return=0:detect_leaks=0:abort_on_error=1",
               **(env_extra or {}))
    r = subprocess.run(["timeout", "-k", "10", "600", driver, str(inp), str(outp)], capture_output=True,
                       text=True, env=env)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-6000:]
    raw = outp.read_bytes()
    status = struct.unpack_from("<i", raw, 0)[0]
    assert status == 0, (status, r.stderr[-2000:])
    if mode == 2:
        return struct.unpack_from("<ff", raw, 4)
    if mode == 4:
        return np.frombuffer(raw, np.float32, n * fmt, 4).reshape(n, fmt)
    nb = struct.unpack_from("<q", raw, 4)[0]
    out = np.frombuffer(raw, np.uint8, nb, 12)
    guard_ok, recounts = struct.unpack_from("<iq", raw, 12 + nb)
    assert guard_ok == 1, "write past the output"
    return out.view(O.FMT_DTYPE[fmt]), recounts


def forest(seed, n, t, nleaf, p_oob=0.368, p_invalid=0.0):
    rng = np.random.default_rng(seed)
    leaf = rng.integers(0, nleaf, size=(t, n)).astype(np.int32)
    if p_invalid:
        bad = rng.random((t, n)) < p_invalid
        leaf[bad] = rng.choice(np.array([-1, nleaf, nleaf + 7], np.int32), size=int(bad.sum()))
    oob = (rng.random((t, n)) < p_oob).astype(np.uint8)
    return leaf, oob


@pytest.mark.parametrize("fmt,scale,zp", [(O.FMT_U16, 1.0, 0.0), (O.FMT_F32, 1.0, 0.0), (O.FMT_F16, 1.0, 0.0),
                                          (O.FMT_NF4, 1.0, 0.0), (O.FMT_U8, 1 / 255.0, 0.0),
                                          (O.FMT_U8, 1 / 4000.0, 3.0), (O.FMT_I8, 1 / 2000.0, -100.0)])
def test_whole_tree_path_every_format(driver, tmp_path, fmt, scale, zp):
    leaf, oob = forest(3, 700, 40, 23, p_invalid=0.02)
    got, _ = emulate(driver, tmp_path, 1, leaf, oob, 23, fmt, scale, zp)
    want = O.upper_rows(leaf, oob, 23, fmt, scale=np.float32(scale), zp=np.float32(zp))
    assert np.array_equal(got, want)


def test_byte_sum_check_and_recount(driver, tmp_path):
    # T = 700 turns on the 8-bit wrap check; samples 0..59 share a leaf in
    # every tree, so their counts (~350) wrap and their items are recounted
    leaf, oob = forest(4, 600, 700, 30, p_oob=0.5)
    leaf[:, :60] = leaf[:, :1]
    for fmt, scale in ((O.FMT_U16, 1.0), (O.FMT_U8, 1 / 255.0)):
        got, rec = emulate(driver, tmp_path, 1, leaf, oob, 30, fmt, scale)
        assert np.array_equal(got, O.upper_rows(leaf, oob, 30, fmt, scale=np.float32(scale)))
        assert rec > 0


# one format per epilogue: the integer deferred codes (U8; I8 shares them),
# the NF4 kernel's, and the float entries (F32; F16 shares them)
@pytest.mark.parametrize("fmt,scale,zp", [(O.FMT_U8, 1 / 4000.0, 3.0), (O.FMT_NF4, 1.0, 0.0), (O.FMT_F32, 1.0, 0.0)])
def test_wrapped_last_column_reads_no_entry_past_the_row(driver, tmp_path, fmt, scale, zp):
    """Checked 8-bit counting (T = 700) where the last column of many rows
    wraps: samples 0..299 and N - 1 share a leaf in every tree, so pairs
    (i, N - 1) count about 325.  The wrap's carry lands in the first padding
    byte after the row's last column; the epilogue must not code that byte
    (whose column N does not exist: its 1/nout would be read past the end of
    the array, which the sanitizer reports).  Column-dependent codes (every
    nonzero count takes the exact per-column path) and a caller nout with
    zeros for the integer formats; the float formats read r_j for every
    nonzero count.  Rows 0..23 (items of different alignments) against the
    oracle after the 16-bit recount."""
    n, t, nleaf = 1003, 700, 3
    leaf, oob = forest(31, n, t, nleaf, p_oob=0.45)
    leaf[:, :300] = leaf[:, :1]
    leaf[:, n - 1] = leaf[:, 0]
    nout = np.random.default_rng(32).integers(0, t + 3, n).astype(np.int32)
    nout[::11] = 0
    got, rec = emulate(driver, tmp_path, 1, leaf, oob, nleaf, fmt, scale, zp, r0=0, r1=24, nout=nout)
    want = O.upper_rows(leaf, oob, nleaf, fmt, scale=np.float32(scale), zp=np.float32(zp), r0=0, r1=24,
                        nout_arr=nout)
    assert np.array_equal(got, want)
    assert rec > 0


@pytest.mark.parametrize("planted", [True, False])
def test_thousand_trees_per_thread_dummy_words(driver, tmp_path, planted):
    """T = 1,000 (769 to 3,072 trees: the byte-sum check with one dummy word
    per thread) on row bands at both ends.  Planted: samples 0..99 share a
    leaf in every tree, their counts (~465) wrap 8 bits and their items are
    recounted; otherwise no item is."""
    n, t = 1500, 1000
    nleaf = 40 if planted else 200
    leaf, oob = forest(97 + planted, n, t, nleaf, p_oob=0.368)
    if planted:
        leaf[:, :100] = leaf[:, :1]
    runs = [(0, 12, O.FMT_U16, 1.0)] + ([(0, 12, O.FMT_U8, 1 / 255.0), (n - 9, n, O.FMT_U16, 1.0)] if planted else [])
    for r0, r1, fmt, scale in runs:
        got, rec = emulate(driver, tmp_path, 1, leaf, oob, nleaf, fmt, scale, r0=r0, r1=r1)
        want = O.upper_rows(leaf, oob, nleaf, fmt, scale=np.float32(scale), r0=r0, r1=r1)
        assert np.array_equal(got, want), (r0, fmt)
        assert (rec > 0) == (planted and r0 == 0), (r0, rec)


@pytest.mark.parametrize("n,t,nleaf,bands", [
    (40_000, 10, 400, [(0, 2), (19_999, 20_002), (39_995, 40_000)]),   # per-part path, keys in registers
    (90_000, 4, 150, [(0, 2), (8_527, 8_530), (89_998, 90_000)]),      # rows split into two items
    (40_000, 6, 1, [(0, 2), (25_000, 25_002)]),                        # buckets of 16,383+ members
])
def test_per_part_path_row_bands(driver, tmp_path, n, t, nleaf, bands):
    leaf, oob = forest(5 + n + nleaf, n, t, nleaf, p_invalid=0.01)
    idx = O.RowIndex(leaf, oob, nleaf)
    for r0, r1 in bands:
        for fmt, scale in ((O.FMT_U16, 1.0), (O.FMT_U8, 1 / 255.0)):
            got, _ = emulate(driver, tmp_path, 1, leaf, oob, nleaf, fmt, scale, r0=r0, r1=r1)
            assert np.array_equal(got, idx.rows(fmt, r0, r1, np.float32(scale), np.float32(0.0))), (r0, fmt)
    idx.close()


@pytest.mark.parametrize("n,t,nleaf,bands", [
    (40_000, 10, 400, [(0, 2), (39_995, 40_000)]),
    (90_000, 4, 150, [(8_527, 8_530), (89_998, 90_000)]),
])
def test_per_part_path_back_to_back_placement(driver, tmp_path, n, t, nleaf, bands):
    """Per-part forests whose line-fit layout would pass 2^30 ids (T * the
    padded tree stride) place their buckets back to back, tree stride N: at
    C3's N that takes about 4,500 trees.  The emulation lowers the bound
    (RFXP_FIT_LIMIT = 1) so that these small forests take that placement;
    the counts, the split rows and the OOB-normalised P V through the bucket
    ends stay exact."""
    from emu_session import EmuScript

    env = {"RFXP_FIT_LIMIT": "1"}
    # the bound takes effect: the forest index (the noalloc workspace counts
    # it) shrinks by the line-fit padding
    ws = []
    for extra in (None, env):
        s = EmuScript(driver)
        s.call("rfxp_upper_noalloc_workspace", n, t, nleaf, 0)
        ws.append(s.run(tmp_path, env_extra=extra)[0])
    assert 0 < ws[1] < ws[0], ws
    leaf, oob = forest(15 + n + nleaf, n, t, nleaf, p_invalid=0.01)
    idx = O.RowIndex(leaf, oob, nleaf)
    for r0, r1 in bands:
        for fmt, scale in ((O.FMT_U16, 1.0), (O.FMT_U8, 1 / 255.0)):
            got, _ = emulate(driver, tmp_path, 1, leaf, oob, nleaf, fmt, scale, r0=r0, r1=r1, env_extra=env)
            assert np.array_equal(got, idx.rows(fmt, r0, r1, np.float32(scale), np.float32(0.0))), (r0, fmt)
    idx.close()
    V = np.random.default_rng(23).standard_normal((n, 4)).astype(np.float32)
    Y = emulate(driver, tmp_path, 4, leaf, oob, nleaf, fmt=4, V=V, env_extra=env)
    want = oob_pv_reference(leaf, oob, nleaf, V)
    assert np.linalg.norm(Y - want) / np.linalg.norm(want) < 1e-6


def test_sample_major_layout_and_caller_nout(driver, tmp_path):
    leaf, oob = forest(6, 500, 33, 5, p_invalid=0.05)
    nout = np.random.default_rng(7).integers(0, 4, size=500).astype(np.int32)
    got, _ = emulate(driver, tmp_path, 1, leaf, oob, 5, O.FMT_F32, nout=nout, layout="sample")
    want = O.upper_rows(leaf, oob, 5, O.FMT_F32, nout_arr=nout)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_minmax_and_noalloc(driver, tmp_path):
    leaf, oob = forest(8, 400, 60, 2)
    nout = np.random.default_rng(9).integers(0, 3, size=400).astype(np.int32)
    mn, mx = emulate(driver, tmp_path, 2, leaf, oob, 2, nout=nout)
    tri = O.upper_rows(leaf, oob, 2, O.FMT_F32, nout_arr=nout)
    assert (mn, mx) == (float(tri.min()), float(tri.max())) and mx > 1
    band = tri[O.tri_idx(400, 350, 350):]
    assert emulate(driver, tmp_path, 2, leaf, oob, 2, r0=350, r1=400, nout=nout) == (float(band.min()),
                                                                                      float(band.max()))
    got, _ = emulate(driver, tmp_path, 3, leaf, oob, 2, O.FMT_U8, 1 / 255.0, r0=17, r1=333)
    assert np.array_equal(got, O.upper_rows(leaf, oob, 2, O.FMT_U8, scale=np.float32(1 / 255.0), r0=17, r1=333))


@pytest.mark.parametrize("n,t,nleaf,plan", [
    (600_000, 3, 16, "direct"),     # parts of 75,000 > 65,535 samples
    (200_000, 4, 256, "sorted2"),   # 2-byte staging keeps two workgroups per CU
    (200_000, 3, 2048, "sorted4"),  # parts of 25,000: keys read twice
    (140_000, 3, 4096, "sorted4"),  # 8,192 buckets
])
def test_member_scatter_variants_row_bands(driver, tmp_path, n, t, nleaf, plan):
    import rfxprox as R

    assert R.pack_plan(n, t, nleaf) == {"direct": R.PACK_PARTS_DIRECT, "sorted2": R.PACK_PARTS_SORTED2,
                                        "sorted4": R.PACK_PARTS_SORTED4}[plan]
    leaf, oob = forest(11 + nleaf, n, t, nleaf, p_invalid=0.02)
    idx = O.RowIndex(leaf, oob, nleaf)
    for r0 in (0, n // 2 - 1, n - 3):
        got, _ = emulate(driver, tmp_path, 1, leaf, oob, nleaf, O.FMT_U16, r0=r0, r1=r0 + 3)
        assert np.array_equal(got, idx.rows(O.FMT_U16, r0, r0 + 3, 1.0, 0.0)), r0
    idx.close()


def oob_pv_reference(leaf, oob, nleaf, V):
    """P V for the cpu_finishprox matrix P = 1/4 (D^-1 U + U D^-1) + I in
    double, U applied per tree through bucket sums: (U X)_i is the sum of X
    over the samples of i's leaf with the other OOB bit."""
    t, n = leaf.shape
    X2 = np.concatenate([V, V], axis=1).astype(np.float64)
    nout = oob.sum(axis=0)
    r = np.where(nout > 0, 1.0 / np.maximum(nout, 1), 1.0)
    X2[:, V.shape[1]:] *= r[:, None]
    Z = np.zeros_like(X2)
    for k in range(t):
        lv = leaf[k].astype(np.int64)
        ok = (lv >= 0) & (lv < nleaf)
        key = np.where(ok, 2 * lv + oob[k], 0)
        S = np.zeros((2 * nleaf, X2.shape[1]))
        np.add.at(S, key[ok], X2[ok])
        Z[ok] += S[key[ok] ^ 1]
    c = V.shape[1]
    return 0.25 * (r[:, None] * Z[:, :c] + Z[:, c:]) + V.astype(np.float64)


@pytest.mark.parametrize("n,t,nleaf", [(900, 20, 7),       # whole-tree path: buckets end where the next starts
                                       (40_000, 5, 300)])  # per-part path: bucket ends from their own table
def test_oob_normalised_pv(driver, tmp_path, n, t, nleaf):
    leaf, oob = forest(21 + n, n, t, nleaf, p_invalid=0.01)
    V = np.random.default_rng(22).standard_normal((n, 8)).astype(np.float32)
    Y = emulate(driver, tmp_path, 4, leaf, oob, nleaf, fmt=8, V=V)
    want = oob_pv_reference(leaf, oob, nleaf, V)
    assert np.linalg.norm(Y - want) / np.linalg.norm(want) < 1e-6


@pytest.mark.parametrize("shape", [("100000", "500", "2048"),           # C3: per-part path
                                   ("140000", "6", "4096", "0.02", "7"),  # 8,192 buckets, invalid labels
                                   ("60000", "20", "2", "0", "5"),        # buckets past 16,383 members
                                   ("40000", "30", "1000", "0.01", "3")])
def test_line_fit_layout_host_check(driver, shape):
    """The line-fit placement at full size, computed on the host with the
    kernels' own rule and stride bound (tests/harness/layout_check.cpp):
    buckets in order inside their tree's stride, small buckets in one line,
    large ones ending on a line, every part's slots and every sample's run
    inside its bucket, long-bucket entries inside mem."""
    r = subprocess.run([os.path.join(EMU, "_build", "layout_check"), *shape], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr
    lines = float(r.stdout.split("lines_per_run=")[1].split()[0])
    assert lines < 1.1 if shape[2] != "2" else True


# ---- the symmetric accumulator behind the low-rank class (rfxp_symacc_*) ----

def _sym(upper_vals, n):
    d = np.zeros((n, n))
    d[np.triu_indices(n)] = upper_vals
    return d + np.triu(d, 1).T


def _values(fmt, data, n, scale=1.0, zp=0.0):
    """Entries i <= j of a contribution as the accumulator reads them
    (cuda/rf_proximity_lowrank.cu:199-240, 654-685, 744-789): FP16 as is, F32
    as is, INT8 and NF4 dequantised then rounded to FP16, a dense double
    matrix's upper triangle rounded through float to FP16."""
    ne = n * (n + 1) // 2
    if fmt == O.FMT_F16:
        return data.view(np.float16).astype(np.float64)
    if fmt == O.FMT_F32:
        return data.astype(np.float64)
    if fmt == O.FMT_I8:
        v = (data.astype(np.float32) - np.float32(zp)) * np.float32(scale)
        return v.astype(np.float16).astype(np.float64)
    if fmt == O.FMT_NF4:
        nib = np.stack([data & 15, data >> 4], axis=1).ravel()[:ne].astype(np.int64)
        v = np.where(nib <= 7, nib.astype(np.float32) / np.float32(7), -(nib - 8).astype(np.float32) / np.float32(7))
        return v.astype(np.float16).astype(np.float64)
    return data[np.triu_indices(n)].astype(np.float32).astype(np.float16).astype(np.float64)


def emulate_symacc(driver, tmp_path, n, contribs, X, rank=0, iters=0):
    """contribs: (fmt or -1 for dense, array, on_device, scale, zp).  Returns
    per add (nnz, device bytes, M X) and, with rank, (A N x rank, Ritz values)."""
    b = X.shape[1]
    inp, outp = tmp_path / "sa_in.bin", tmp_path / "sa_out.bin"
    with open(inp, "wb") as f:
        f.write(struct.pack("<iqiiii", 5, n, len(contribs), b, rank, iters))
        for fmt, arr, on_dev, scale, zp in contribs:
            raw = np.ascontiguousarray(arr).tobytes()
            f.write(struct.pack("<iiffq", fmt, int(on_dev), np.float32(scale), np.float32(zp), len(raw)))
            f.write(raw)
        np.ascontiguousarray(X, np.float64).tofile(f)
    env = dict(os.environ, ASAN_OPTIONS="detect_stack_use_after_return=0:detect_leaks=0:abort_on_error=1")
    r = subprocess.run(["timeout", "-k", "10", "600", driver, str(inp), str(outp)], capture_output=True,
                       text=True, env=env)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-6000:]
    raw = outp.read_bytes()
    assert struct.unpack_from("<i", raw, 0)[0] == 0, r.stderr[-2000:]
    off, steps = 4, []
    for _ in contribs:
        nnz, nbytes = struct.unpack_from("<qq", raw, off)
        Y = np.frombuffer(raw, np.float64, n * b, off + 16).reshape(n, b)
        steps.append((nnz, nbytes, Y))
        off += 16 + 8 * n * b
    if not rank:
        return steps, None
    A = np.frombuffer(raw, np.float64, n * rank, off).reshape(rank, n).T
    ev = np.frombuffer(raw, np.float64, rank, off + 8 * n * rank)
    return steps, (A, ev)


def _check_steps(steps, contribs, n, X):
    ne = n * (n + 1) // 2
    limit = ne // 7 * 2                 # largest list of the sparse form
    M = np.zeros((n, n))
    listed, dense = 0, False
    for (nnz, nbytes, Y), (fmt, arr, _, scale, zp) in zip(steps, contribs):
        v = _values(fmt, arr, n, scale, zp)
        M += _sym(v, n)
        listed += int((v != 0).sum())
        dense = dense or listed > limit
        assert nnz == (ne if dense else listed)
        # the bound: the triangle in doubles, three N + 1 count arrays, one
        # staging buffer (at most 256 bytes in this build, or one row of a
        # dense input and a byte, in 8-byte words)
        stage = -(-max(256, 8 * n + 1) // 8) * 8
        assert nbytes <= 8 * ne + 24 * (n + 1) + stage, (nbytes, 8 * ne)
        want = M @ X
        assert np.abs(Y - want).max() <= 1e-12 * np.abs(M).sum(axis=1).max() * np.abs(X).max()
    return M


def test_symacc_sparse_then_dense(driver, tmp_path):
    """Sparse contributions in host and device memory, then one whose early
    rows are sparse and later rows dense, so that the list passes its limit
    within a contribution and the accumulator changes form between two
    staged bands; then dense-form adds from host (one row per band) and
    device memory.  M X after every add against the dense sum; the
    full-rank factor against numpy's eigendecomposition."""
    rng = np.random.default_rng(51)
    n = 45
    ne = n * (n + 1) // 2
    f16 = np.zeros(ne, np.float16)
    hit = rng.random(ne) < 0.05
    f16[hit] = rng.standard_normal(int(hit.sum())).astype(np.float16)
    q8 = np.full(ne, 3, np.int8)
    hit = rng.random(ne) < 0.08
    q8[hit] = rng.integers(-128, 128, int(hit.sum()))
    rows = np.repeat(np.arange(n), np.arange(n, 0, -1))
    f32 = rng.standard_normal(ne).astype(np.float32)
    f32[(rows < 25) & (rng.random(ne) < 0.9)] = 0      # sparse early rows, dense late rows
    p4 = rng.integers(0, 256, (ne + 1) // 2).astype(np.uint8)
    full = rng.standard_normal((n, n))
    f16b = rng.standard_normal(ne).astype(np.float16)
    contribs = [(O.FMT_F16, f16.view(np.uint16), False, 1.0, 0.0),
                (O.FMT_I8, q8, True, 0.01, 3.0),
                (O.FMT_F32, f32, False, 1.0, 0.0),
                (O.FMT_NF4, p4, False, 1.0, 0.0),
                (-1, full, False, 1.0, 0.0),
                (O.FMT_F16, f16b.view(np.uint16), True, 1.0, 0.0)]
    X = rng.standard_normal((n, 70))                  # two column tiles of the dense product
    steps, (A, ev) = emulate_symacc(driver, tmp_path, n, contribs, X, rank=n, iters=3)
    assert steps[1][0] < ne and steps[2][0] == ne     # the switch came within the F32 add
    M = _check_steps(steps, contribs, n, X)
    w, V = np.linalg.eigh(M)
    w = np.maximum(w, 0.0)
    want = (V * w) @ V.T
    assert np.linalg.norm(A @ A.T - want) <= 1e-9 * np.linalg.norm(want)
    assert np.allclose(np.sort(np.maximum(ev, 0))[::-1], np.sort(w)[::-1], atol=1e-9 * w.max())


def test_symacc_stays_sparse(driver, tmp_path):
    """Contributions that never reach the list's limit: the CSR product and
    the factor of the sparse form."""
    rng = np.random.default_rng(52)
    n = 130
    ne = n * (n + 1) // 2
    contribs = []
    for k in range(4):
        f16 = np.zeros(ne, np.float16)
        hit = rng.random(ne) < 0.04
        f16[hit] = rng.standard_normal(int(hit.sum())).astype(np.float16)
        contribs.append((O.FMT_F16, f16.view(np.uint16), bool(k % 2), 1.0, 0.0))
    X = rng.standard_normal((n, 5))
    steps, (A, ev) = emulate_symacc(driver, tmp_path, n, contribs, X, rank=n, iters=3)
    assert steps[-1][0] < ne // 7 * 2
    M = _check_steps(steps, contribs, n, X)
    w, V = np.linalg.eigh(M)
    w = np.maximum(w, 0.0)
    want = (V * w) @ V.T
    assert np.linalg.norm(A @ A.T - want) <= 1e-9 * np.linalg.norm(want)


def test_symacc_dense_from_the_first_add(driver, tmp_path):
    """A first contribution denser than the limit: the dense form from the
    start (empty list), host NF4 bands that start at odd entries."""
    rng = np.random.default_rng(53)
    n = 77
    ne = n * (n + 1) // 2
    p4 = rng.integers(0, 256, (ne + 1) // 2).astype(np.uint8)
    full = rng.standard_normal((n, n))
    contribs = [(O.FMT_NF4, p4, False, 1.0, 0.0), (-1, full, True, 1.0, 0.0), (O.FMT_NF4, p4, True, 1.0, 0.0)]
    X = rng.standard_normal((n, 3))
    steps, _ = emulate_symacc(driver, tmp_path, n, contribs, X)
    assert steps[0][0] == ne
    _check_steps(steps, contribs, n, X)


def test_symacc_list_scan_over_row_chunks(driver, tmp_path):
    """N = 2,500 rows in one band: the device scan of the row counts gives
    each of its 1,024 threads a chunk of three rows."""
    rng = np.random.default_rng(54)
    n = 2500
    ne = n * (n + 1) // 2
    contribs = []
    for k in range(2):
        f16 = np.zeros(ne, np.float16)
        hit = rng.random(ne) < 0.002
        f16[hit] = rng.standard_normal(int(hit.sum())).astype(np.float16)
        contribs.append((O.FMT_F16, f16.view(np.uint16), True, 1.0, 0.0))
    X = rng.standard_normal((n, 3))
    steps, _ = emulate_symacc(driver, tmp_path, n, contribs, X)
    assert 0 < steps[-1][0] < ne // 7 * 2
    _check_steps(steps, contribs, n, X)


SWEEP_FMTS = [(O.FMT_U16, 1.0, 0.0), (O.FMT_F32, 1.0, 0.0), (O.FMT_F16, 1.0, 0.0), (O.FMT_U8, 1 / 255.0, 0.0),
              (O.FMT_U8, 1 / 4000.0, 3.0), (O.FMT_I8, 1 / 127.0, 0.0), (O.FMT_I8, 1 / 2000.0, -100.0),
              (O.FMT_NF4, 1.0, 0.0)]


def random_case(seed):
    """One random forest shape of the triangle sweep: N up to 130,000 (row
    bands for large N), T up to 1,200, leaves from 1 to 20,000 (both packing
    paths), any OOB rate, invalid labels, blocks of samples sharing leaves,
    either layout, caller nout or not, every format."""
    rng = np.random.default_rng(seed)
    big = rng.random() < 0.15
    n = int(rng.integers(40000, 130000)) if big else int(rng.integers(1, 3000))
    t = int(rng.integers(1, 8)) if big else int(rng.choice([1, 2, 3, 17, 64, 255, 256, 300, 700, 1000,
                                                             int(rng.integers(1, 1200))]))
    nleaf = int(rng.choice([1, 2, 3, 50, 400, 2048, 4096, 4097, 9000, int(rng.integers(1, 20000))]))
    p_oob = float(rng.choice([0.0, 0.37, 1.0, float(rng.random())]))
    p_inv = float(rng.choice([0.0, 0.0, 0.02, 0.3]))
    leaf, oob = forest(seed, n, t, nleaf, p_oob=p_oob, p_invalid=p_inv)
    if rng.random() < 0.3 and n > 10:
        k = int(rng.integers(2, min(n, 300)))
        leaf[:, :k] = leaf[:, :1]
    fmt, scale, zp = SWEEP_FMTS[int(rng.integers(len(SWEEP_FMTS)))]
    if big or rng.random() < 0.4:
        r0 = int(rng.integers(0, n))
        r1 = int(min(n, r0 + rng.integers(1, 6)))
    else:
        r0, r1 = 0, n
    layout = "sample" if rng.random() < 0.3 else "tree"
    nout = rng.integers(0, t + 3, n).astype(np.int32) if rng.random() < 0.25 else None
    return leaf, oob, nleaf, fmt, scale, zp, r0, r1, layout, nout


# chosen from a sweep of ~470 such cases (all bit-exact) to cover both packing
# paths, row bands of large N, both layouts, caller nout and every format
@pytest.mark.parametrize("seed", [100000, 100002, 100005, 100011, 100021, 100033, 100035, 100039, 100055, 100079])
def test_random_shapes(driver, tmp_path, seed):
    leaf, oob, nleaf, fmt, scale, zp, r0, r1, layout, nout = random_case(seed)
    n = leaf.shape[1]
    got, _ = emulate(driver, tmp_path, 1, leaf, oob, nleaf, fmt, scale, zp, r0=r0, r1=r1, nout=nout, layout=layout)
    want = O.upper_rows(leaf, oob, nleaf, fmt, scale=np.float32(scale), zp=np.float32(zp), r0=r0, r1=r1,
                        nout_arr=nout)
    g, w = got.view(np.uint8).copy(), want.view(np.uint8).copy()
    if fmt == O.FMT_NF4 and len(g):   # nibbles of entries outside the rows are the caller's
        if O.tri_idx(n, r0, r0) & 1:
            g[0] &= 0xF0
            w[0] &= 0xF0
        if O.tri_idx(n, r1, r1) & 1:
            g[-1] &= 0x0F
            w[-1] &= 0x0F
    assert np.array_equal(g, w)


@pytest.mark.parametrize("order,lanes,blocks,fill", [("reverse", "forward", "reverse", "0x00"),
                                                     ("shuffle", "reverse", "shuffle", "0xff")])
def test_results_do_not_depend_on_wave_order(driver, tmp_path, monkeypatch, order, lanes, blocks, fill):
    """The emulator runs the waves of a workgroup in reverse or shuffled
    order between synchronization points, the lanes of a wave in reverse
    order and a launch's workgroups in reverse or shuffled order, with fresh
    LDS and device memory holding another byte: a kernel whose waves
    exchange data without a barrier, whose workgroups depend on their order,
    or that reads memory it never wrote would give a different result.  The
    whole-tree and per-part packing paths with the triangle."""
    monkeypatch.setenv("EMU_ORDER", order)
    monkeypatch.setenv("EMU_LANES", lanes)
    monkeypatch.setenv("EMU_BLOCKS", blocks)
    monkeypatch.setenv("EMU_FILL", fill)
    monkeypatch.setenv("EMU_SEED", "11")
    leaf, oob = forest(12, 400, 260, 9, p_invalid=0.01)    # T > 255: the byte-sum check runs
    leaf[:, :40] = leaf[:, :1]
    got, _ = emulate(driver, tmp_path, 1, leaf, oob, 9, O.FMT_U8, 1 / 255.0)
    assert np.array_equal(got, O.upper_rows(leaf, oob, 9, O.FMT_U8, scale=np.float32(1 / 255.0)))
    leaf, oob = forest(13, 40_000, 6, 300)
    got, _ = emulate(driver, tmp_path, 1, leaf, oob, 300, O.FMT_U16, r0=19_998, r1=20_001)
    assert np.array_equal(got, O.upper_rows(leaf, oob, 300, O.FMT_U16, r0=19_998, r1=20_001))
