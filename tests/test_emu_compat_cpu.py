"""The per-tree and dense small-N functions (rfxp_tree_accumulate,
rfxp_tree_pairs, rfxp_finishprox, rfxp_rfgap, rfxp_tree_upper,
rfxp_rfgap_tree_upper): the library's kernels run on the CPU by the
emulator (tests/emu, script mode), through the C ABI, against the
reference's golden fixtures (tests/golden) and the oracle, bit-exact, with
host and device inputs and outputs."""
import os

import numpy as np
import pytest

import oracle as O
from emu_session import CTX, EmuScript

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def fixture():
    g = np.load(os.path.join(GOLD, "cpu_prox_small.npz"))
    return (g["nodestatus"].astype(np.int32), g["nodextr"].astype(np.int32), g["nin"].astype(np.int32), g)


def random_tree(rng, n, nnode, p_term=0.7, oob=0.37):
    ns = np.where(rng.random(nnode) < p_term, -1, rng.integers(1, 3, nnode)).astype(np.int32)
    nx = rng.integers(-2, nnode + 2, n).astype(np.int32)
    nin = np.bincount(rng.integers(0, n, n), minlength=n).astype(np.int32)
    nin[rng.random(n) < oob - 0.37] = 0
    return ns, nx, nin


def tree_args(s, ns, nx, nin, on_device):
    put = s.dev if on_device else s.host
    return put(ns), put(nx), put(nin)


@pytest.mark.parametrize("cw", [0, 1])
def test_accumulate_and_finishprox_reference_fixture(emu_driver, tmp_path, cw):
    ns, nx, nin, g = fixture()
    t, n = nx.shape
    s = EmuScript(emu_driver)
    prox = s.host(np.zeros(n * n), want=True)
    for k in range(t):
        s.call("rfxp_tree_accumulate", CTX, *tree_args(s, ns[k], nx[k], nin[k], k % 2), n, ns.shape[1], cw, prox)
    sym = s.out(8 * n * n, host=True)
    s.call("rfxp_finishprox", CTX, n, s.host(g["nout"].astype(np.int32)), prox, sym)
    sym_d = s.out(8 * n * n)
    s.call("rfxp_finishprox", CTX, n, s.dev(g["nout"].astype(np.int32)), s.dev(g[f"prox_cw{cw}"]), sym_d)
    assert s.run(tmp_path) == [0] * (t + 2)
    F = lambda b: b.array(np.float64).reshape((n, n), order="F")  # noqa: E731
    assert np.array_equal(F(prox), g[f"prox_cw{cw}"])
    assert np.array_equal(F(sym), g[f"proxsym_cw{cw}"])
    assert np.array_equal(F(sym_d), g[f"proxsym_cw{cw}"])


@pytest.mark.parametrize("n,nnode,seed", [(1, 1, 0), (37, 5, 1), (700, 40, 2)])
def test_accumulate_random_trees(emu_driver, tmp_path, n, nnode, seed):
    rng = np.random.default_rng(seed)
    s = EmuScript(emu_driver)
    want = {cw: np.zeros((n, n), order="F") for cw in (0, 1)}
    got = {cw: s.host(np.zeros(n * n), want=True) for cw in (0, 1)}
    npairs = []
    nout = np.zeros(n, np.int32)
    trees = [random_tree(rng, n, nnode) for _ in range(4)]
    for ns, nx, nin in trees:
        nout += nin == 0
        for cw in (0, 1):
            O.cpu_proximity(ns, nx, nin, nnode, want[cw], bool(cw))
            s.call("rfxp_tree_accumulate", CTX, *tree_args(s, ns, nx, nin, cw), n, nnode, cw, got[cw])
        pi, pw, cnt = s.out(8, host=True), s.out(8, host=True), s.out(8, host=True)
        s.call("rfxp_tree_pairs", CTX, *tree_args(s, ns, nx, nin, 0), n, nnode, 1, pi, pw, cnt)
        npairs.append(cnt)
    assert s.run(tmp_path) == [0] * (3 * len(trees))
    for cw in (0, 1):
        assert np.array_equal(got[cw].array(np.float64).reshape((n, n), order="F"), want[cw])
    for (ns, nx, nin), cnt in zip(trees, npairs):
        # one pair per OOB sample in a terminal node of non-zero size, per in-bag member of that node
        node = np.where((nx >= 0) & (nx < nnode), nx, -1)
        term = (node >= 0) & (ns[np.maximum(node, 0)] == -1)
        inbag = term & (nin > 0)
        members = np.bincount(node[inbag], minlength=nnode)
        want_pairs = int(members[node[term & (nin == 0)]].sum())
        assert cnt.array(np.int64)[0] == want_pairs


def test_rfgap_reference_fixture_and_random(emu_driver, tmp_path):
    g = np.load(os.path.join(GOLD, "rfgap_small.npz"))
    rng = np.random.default_rng(2)
    n, t, nnode = 400, 9, 30
    nin = np.stack([np.bincount(rng.integers(0, n, n), minlength=n) for _ in range(t)]).astype(np.int32)
    nx = rng.integers(-1, nnode, (t, n)).astype(np.int32)
    nin[:, 0] = 1                                   # sample 0 never OOB
    s = EmuScript(emu_driver)
    gt, gn = g["nin"].shape
    out_g = s.out(8 * gn * gn, host=True)
    s.call("rfxp_rfgap", CTX, gt, gn, s.host(g["nin"].astype(np.int32)), s.host(g["nodextr"].astype(np.int32)),
           out_g)
    out_r = s.out(8 * n * n)
    s.call("rfxp_rfgap", CTX, t, n, s.dev(nin), s.dev(nx), out_r)
    assert s.run(tmp_path) == [0, 0]
    assert np.array_equal(out_g.array(np.float64).reshape((gn, gn), order="F"), g["prox"])
    assert np.array_equal(out_r.array(np.float64).reshape((n, n), order="F"), O.rfgap(nin, nx))


FMTS = [(O.FMT_F16, 1.0, 0.0), (O.FMT_NF4, 1.0, 0.0), (O.FMT_I8, 1.0 / 127.0, 0.0), (O.FMT_I8, 0.013, -3.5)]


def out_bytes(fmt, m):
    ne = m * (m + 1) // 2
    return {O.FMT_F16: 2 * ne, O.FMT_I8: ne, O.FMT_NF4: (ne + 1) // 2}[fmt]


def test_tree_upper_fixture_and_random_trees(emu_driver, tmp_path):
    """Every per-tree format, casewise or not, on the fixture's trees and on
    random trees (n_real < N included), host and device outputs."""
    ns0, nx0, nin0, _ = fixture()
    rng = np.random.default_rng(3)
    cases = [(ns0[k], nx0[k], nin0[k], 0) for k in range(0, nx0.shape[0], 3)]
    cases += [random_tree(rng, n, nnode) + (n_real,) for n, nnode, n_real in [(1, 1, 0), (2, 1, 0), (333, 7, 0),
                                                                             (1025, 25, 999)]]
    s = EmuScript(emu_driver)
    checks = []
    for c, (ns, nx, nin, n_real) in enumerate(cases):
        n = len(nx)
        m = n_real if 0 < n_real < n else n
        for fmt, scale, zp in FMTS:
            for cw in (0, 1):
                on_dev = (c + cw) % 2
                o = s.out(out_bytes(fmt, m), host=not on_dev)
                s.call("rfxp_tree_upper", CTX, fmt, *tree_args(s, ns, nx, nin, on_dev), n, len(ns), cw, n_real,
                       float(np.float32(scale)), float(np.float32(zp)), o)
                checks.append((o, fmt, ns, nx, nin, cw, n_real, scale, zp))
    assert s.run(tmp_path) == [0] * len(checks)
    for o, fmt, ns, nx, nin, cw, n_real, scale, zp in checks:
        want = O.tree_upper(fmt, ns, nx, nin, casewise=bool(cw), n_real=n_real, scale=scale, zp=zp)
        assert np.array_equal(o.array(want.dtype), want), (fmt, len(nx), cw)


@pytest.mark.parametrize("n", [1000, 1001])
def test_tree_upper_device_output_in_place_or_staged(emu_driver, tmp_path, n):
    """Word-sized device outputs are written in place, others through
    staging; the bytes after the triangle stay as they were."""
    rng = np.random.default_rng(5)
    ns, nx, nin = random_tree(rng, n, 17)
    s = EmuScript(emu_driver)
    outs = []
    for fmt, dt in ((O.FMT_F16, np.uint16), (O.FMT_I8, np.int8), (O.FMT_NF4, np.uint8)):
        nb = out_bytes(fmt, n)
        o = s.dev(np.full((nb + 3) // 4 * 4 + 4, 0xFF, np.uint8), want=True)
        s.call("rfxp_tree_upper", CTX, fmt, *tree_args(s, ns, nx, nin, 0), n, 17, 1, 0, 0.02, 1.0, o)
        outs.append((o, fmt, dt, nb))
    assert s.run(tmp_path) == [0, 0, 0]
    for o, fmt, dt, nb in outs:
        raw = o.array(np.uint8)
        want = O.tree_upper(fmt, ns, nx, nin, casewise=True, scale=np.float32(0.02), zp=1.0)
        assert np.array_equal(raw[:nb].view(dt), want), fmt
        assert (raw[nb:] == 0xFF).all()


@pytest.mark.parametrize("n,n_real,seed", [(1, 0, 0), (80, 0, 1), (1200, 1000, 2)])
def test_rfgap_tree_upper(emu_driver, tmp_path, n, n_real, seed):
    rng = np.random.default_rng(seed)
    nin = np.bincount(rng.integers(0, n, n), minlength=n).astype(np.int32)
    nx = rng.integers(-1, 9, n).astype(np.int32)
    m = n_real if 0 < n_real < n else n
    s = EmuScript(emu_driver)
    o_host = s.out(2 * (m * (m + 1) // 2), host=True)
    o_dev = s.out(2 * (m * (m + 1) // 2))
    s.call("rfxp_rfgap_tree_upper", CTX, s.host(nin), s.host(nx), n, n_real, o_host)
    s.call("rfxp_rfgap_tree_upper", CTX, s.dev(nin), s.dev(nx), n, n_real, o_dev)
    assert s.run(tmp_path) == [0, 0]
    want = O.rfgap_tree_upper(nin, nx, n_real=n_real)
    assert np.array_equal(o_host.array(np.uint16), want)
    assert np.array_equal(o_dev.array(np.uint16), want)


def test_bad_arguments_are_errors(emu_driver, tmp_path):
    ns, nx, nin, _ = fixture()
    s = EmuScript(emu_driver)
    z = s.host(np.zeros(4, np.int32))
    s.call("rfxp_finishprox", CTX, -1, z, z, z)
    s.call("rfxp_tree_upper", CTX, O.FMT_F16, s.host(ns[0]), s.host(nx[0]), s.host(nin[0]), nx.shape[1],
           ns.shape[1], 0, 0, 1.0, 0.0, None)
    s.call("rfxp_rfgap", CTX, 2, -5, z, z, z)
    s.call("rfxp_tree_upper", CTX, 17, s.host(ns[0]), s.host(nx[0]), s.host(nin[0]), nx.shape[1], ns.shape[1], 0,
           0, 1.0, 0.0, s.out(64, host=True))
    assert s.run(tmp_path) == [1, 1, 1, 5]          # RFXP_ERR_INVALID x 3, then an unsupported format
