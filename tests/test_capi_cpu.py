"""CPU-side checks of the product library: it loads, exports every function
that include/rfx_prox.h declares, its host-only helpers compute the right
sizes, and without a GPU it fails with an error instead of falling back."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import rfxprox as R

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_function():
    lib = R.load()
    names = R.header_functions()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_exported_symbols_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", R.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    for n in R.header_functions():
        assert f" T {n}\n" in out + "\n" or f" T {n}" in out


def test_upper_nbytes():
    N = 100_000
    assert R.upper_nbytes(R.FMT_U8, N) == N * (N + 1) // 2 == 5_000_050_000
    assert R.upper_nbytes(R.FMT_F32, 20_000) == 4 * 200_010_000
    assert R.upper_nbytes(R.FMT_U16, 7) == 2 * 28
    # NF4: bytes touched by entries [e0, e1)
    assert R.upper_nbytes(R.FMT_NF4, 5) == 8          # 15 entries
    assert R.upper_nbytes(R.FMT_NF4, 5, 1, 3) == 4    # entries 5..11 -> bytes 2..5
    with pytest.raises(ValueError):
        R.upper_nbytes(R.FMT_U8, 10, 5, 4)
    with pytest.raises(ValueError):
        R.upper_nbytes(17, 10)


def test_no_device_is_an_error_not_a_fallback():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(R.RfxpError):
        R.Context(0)
    buf = ctypes.create_string_buffer(256)
    R.load().rfxp_last_error(None, buf, 256)
    assert b"no HIP device" in buf.value


COMPAT_HDR = os.path.join(REPO, "include", "rfx_compat.hpp")


def compat_functions():
    """Function names declared in include/rfx_compat.hpp (reference signatures),
    the inline device converters excluded."""
    import re

    src = open(COMPAT_HDR).read()
    names = re.findall(r"^\s*(?:static\s+)?(?:void|size_t|__global__\s+void)\s+(\w+)\(", src, re.M)
    return sorted(set(names) - {"rfx_compat_configure"})


def test_library_exports_reference_signatures():
    out = subprocess.run(["nm", "-DC", "--defined-only", R.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    names = compat_functions()
    assert {"cpu_proximity", "gpu_proximity_upper_triangle_int8", "get_quantized_size",
            "cuda_proximity_nf4_kernel"} <= set(names)
    for n in names:
        assert f"::{n}(" in out, f"{n} declared in rfx_compat.hpp, not exported"
    assert " T rfx_compat_configure" in out and " T rfx_compat_last_error" in out
    # the C++ entry points keep the reference's parameter types
    assert "rf::cpu_proximity(int const*, int const*, int const*, int, int, double*, int*, int*, int*, int*, " \
           "int*, int*)" in out
    assert "rf::cpu_proximity_rfgap(int, int, std::vector<std::vector<int, std::allocator<int> >" in out


def test_compat_entry_without_device_reports_error_and_leaves_output():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    lib = ctypes.CDLL(R.LIB_PATH)
    lib.rfx_compat_last_error.restype = ctypes.c_char_p
    # rf::cpu_finishprox(int, const int*, double*, double*) by its mangled name
    fn = getattr(lib, "_ZN2rf14cpu_finishproxEiPKiPdS2_")
    n = 3
    nout = (ctypes.c_int32 * n)(1, 1, 1)
    prox = (ctypes.c_double * (n * n))(*([0.5] * 9))
    sym = (ctypes.c_double * (n * n))(*([7.0] * 9))
    fn(ctypes.c_int32(n), nout, prox, sym)
    assert list(sym) == [7.0] * 9
    assert b"no HIP device" in lib.rfx_compat_last_error()


def test_host_int8_scaling_matches_reference_formula_and_rejects_empty_input():
    """rf::cuda::QuantizationUtils::compute_int8_scaling is host code: scale =
    (max - min)/255, zero_point = -min/scale in float
    (cuda/rf_quantization_kernels.cu:107-119); an empty input is reported and
    leaves the outputs as they were (the reference reads data[0] regardless)."""
    import numpy as np

    lib = ctypes.CDLL(R.LIB_PATH)
    lib.rfx_compat_last_error.restype = ctypes.c_char_p
    fn = getattr(lib, "_ZN2rf4cuda17QuantizationUtils20compute_int8_scalingEPKfmRfS4_")
    fn.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
    data = np.array([0.25, -0.5, 0.75, 0.1], dtype=np.float32)
    sc, zp = ctypes.c_float(0), ctypes.c_float(0)
    fn(data.ctypes.data, data.size, ctypes.byref(sc), ctypes.byref(zp))
    want_sc = (np.float32(0.75) - np.float32(-0.5)) / np.float32(255.0)
    assert sc.value == want_sc and zp.value == np.float32(-np.float32(-0.5) / want_sc)
    sc, zp = ctypes.c_float(3.0), ctypes.c_float(4.0)
    fn(data.ctypes.data, 0, ctypes.byref(sc), ctypes.byref(zp))
    assert (sc.value, zp.value) == (3.0, 4.0)
    assert b"no data" in lib.rfx_compat_last_error()


def _all_segments(n, s, r0, r1):
    """Every (row, first column) segment of rows [r0, r1): segment k of row i
    starts at i + k*S while N - i > k*S."""
    return {(i, i + k * s) for i in range(r0, r1) for k in range((n - i + s - 1) // s)}


@pytest.mark.parametrize("n,s,r0,r1", [(1, 1, 0, 1), (5, 2, 0, 5), (5, 2, 1, 3), (17, 4, 0, 17),
                                       (17, 4, 16, 17), (100, 7, 3, 98), (100, 100, 0, 100),
                                       (100, 1000, 0, 100), (1000, 77, 0, 1000), (1000, 77, 500, 501),
                                       (999, 64, 937, 999), (64, 64, 0, 1), (300, 41, 9, 290)])
def test_upper_work_items_cover_the_band_once(n, s, r0, r1):
    """Slots of rfxp_upper's decomposition: the non-idle ones cover every
    segment of the band exactly once; all segments of a row sit on slots
    congruent mod 8 (one XCD), in increasing column order one slot-group of
    8 apart; each segment's output range lies inside the band's buffer."""
    slots = R.upper_work_items(n, s, r0, r1)
    assert len(slots) % 8 == 0
    real = [(b, i, lo) for b, (i, lo) in enumerate(slots) if i >= 0]
    assert len({(i, lo) for _, i, lo in real}) == len(real)
    assert {(i, lo) for _, i, lo in real} == _all_segments(n, s, r0, r1)
    by_row = {}
    for b, i, lo in real:
        assert b % 8 == (i - r0) % 8
        by_row.setdefault(i, []).append((b, lo))
    for i, lst in by_row.items():
        lst.sort()
        assert [lo for _, lo in lst] == [i + k * s for k in range(len(lst))]
        assert all(b1 - b0 == 8 for (b0, _), (b1, _) in zip(lst, lst[1:]))
    e_base = r0 * n - r0 * (r0 + 1) // 2 + r0
    e_end = r1 * n - r1 * (r1 + 1) // 2 + r1
    covered = 0
    for _, i, lo in real:
        width = min(s, n - lo)
        e0 = i * n - i * (i + 1) // 2 + lo
        assert e_base <= e0 and e0 + width <= e_end
        covered += width
    assert covered == e_end - e_base
    # idle slots are a small share
    assert len(slots) - len(real) <= 8 * ((n - r0 + s - 1) // s) + 7


def test_upper_work_items_at_large_sizes():
    """Closed form at sizes where enumeration is too long: slot counts, a
    sample of slots, and the launch split at 2^22 - 8 workgroups."""
    L = R.load()
    import ctypes as C

    row, col = C.c_int64(), C.c_int64()
    n, s = 100_000, 77_696
    cnt = L.rfxp_upper_work_item(n, s, 0, n, -1, None, None)
    # groups of 8 rows: two segments while the group's first row is below N - S
    g2 = (n - s + 7) // 8
    assert cnt == 8 * ((n + 7) // 8) + 8 * g2
    n = 5_000_000
    cnt = L.rfxp_upper_work_item(n, s, 0, n, -1, None, None)
    segs = sum(max(0, n - k * s) for k in range((n + s - 1) // s))
    assert segs <= cnt <= segs + 8 * 65 and cnt > (1 << 22)
    big = (1 << 22) - 8
    assert L.rfxp_upper_launches(cnt) == (cnt + big - 1) // big
    assert L.rfxp_upper_launches(big) == 1 and L.rfxp_upper_launches(big + 1) == 2
    for e in (0, 1, 8, cnt // 3, cnt // 2, cnt - 9, cnt - 1):
        L.rfxp_upper_work_item(n, s, 0, n, e, C.byref(row), C.byref(col))
        i, lo = row.value, col.value
        if i >= 0:
            assert 0 <= i <= lo < n and (lo - i) % s == 0 and e % 8 == i % 8
    assert L.rfxp_upper_work_item(n, s, 7, 3, 0, None, None) == -1


def test_outlier_normalize_host_matches_oracle():
    """rfxp_outlier_normalize is host-only: it runs without a device."""
    import oracle as O

    rng = np.random.default_rng(3)
    raw = rng.gamma(2.0, 3.0, 1001).astype(np.float32)
    cls = rng.integers(0, 4, 1001).astype(np.int32)
    for c in (None, cls):
        got, med, mad = R.outlier_normalize(raw, c)
        assert np.array_equal(got, O.outlier_normalize(raw, c))
    got, med, mad = R.outlier_normalize(np.array([5, 1, 3, 2, 4], np.float32))
    assert med[0] == 3 and mad[0] == 1


@pytest.mark.parametrize("n,seed", [(1, 0), (7, 1), (40, 2), (130, 3)])
def test_host_symeig_matches_numpy(n, seed):
    """The host eigensolver of the factor and MDS paths (cyclic Jacobi)
    against numpy.linalg.eigh, including repeated eigenvalues."""
    import ctypes as C

    rng = np.random.default_rng(seed)
    a = rng.standard_normal((n, n))
    a = a + a.T
    if n >= 7:  # a repeated eigenvalue and a zero one
        q, _ = np.linalg.qr(rng.standard_normal((n, n)))
        lam = rng.standard_normal(n)
        lam[1] = lam[0]
        lam[2] = 0.0
        a = (q * lam) @ q.T
        a = 0.5 * (a + a.T)
    L = R.load()
    L.rfxp_host_symeig.argtypes = [C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]
    A = np.ascontiguousarray(a)
    w = np.empty(n)
    v = np.empty((n, n))
    assert L.rfxp_host_symeig(n, A.ctypes.data, w.ctypes.data, v.ctypes.data) == 0
    want = np.sort(np.linalg.eigvalsh(a))[::-1]
    scale = max(1.0, np.abs(want).max())
    assert np.allclose(w, want, rtol=0, atol=1e-12 * scale)
    assert np.allclose(v.T @ v, np.eye(n), atol=1e-12)
    assert np.allclose(a @ v, v * w, atol=1e-11 * scale)


def test_library_exports_lowrank_class_with_reference_signatures():
    """include/rf_proximity_lowrank.hpp:27-433 and rf_lowrank_helpers.hpp:13-34:
    every public member and helper, with the reference's parameter types."""
    out = subprocess.run(["nm", "-DC", "--defined-only", R.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    C_ = "rf::cuda::LowRankProximityMatrix::"
    want = [
        C_ + "LowRankProximityMatrix(int, int, rf::cuda::QuantizationLevel, int, int)",
        C_ + "~LowRankProximityMatrix()",
        C_ + "initialize()",
        C_ + "add_tree_contribution(double const*, int, bool)",
        C_ + "add_tree_contribution_incremental(double const*, int)",
        C_ + "add_tree_contribution_incremental_upper_triangle(void const*, int, rf::cuda::QuantizationLevel, "
             "float, float)",
        C_ + "add_tree_contribution_incremental_upper_triangle_fp16(__half const*, int)",
        C_ + "finalize_accumulation(int, bool)",
        C_ + "get_accumulated_proximity(double*, int)",
        C_ + "reconstruct_full_matrix(double*, int, rf::cuda::QuantizationLevel)",
        C_ + "quantize_factors(rf::cuda::QuantizationLevel)",
        C_ + "dequantize_factors()",
        C_ + "get_factors(double**, double**, int*)",
        C_ + "compute_distances_from_factors(double*, int)",
        C_ + "set_oob_counts_for_rfgap(int const*)",
        C_ + "compute_mds_from_factors(int)",
        C_ + "auto_adjust_rank(double)",
        C_ + "get_memory_usage() const",
        C_ + "get_memory_usage(rf::cuda::QuantizationLevel) const",
        C_ + "should_use_incremental(int, unsigned long)",
        "rf::cuda::estimate_optimal_rank(int, int)",
        "rf::cuda::get_lowrank_factors_host(void*, double**, double**, int*, int)",
        "rf::cuda::compute_mds_from_factors_host(void*, int)",
        "rf::cuda::reconstruct_proximity_matrix_host(void*, double**, int)",
    ]
    for w in want:
        assert w in out, w


@pytest.mark.parametrize("args,plan", [
    ((100_000, 500, 2048), R.PACK_PARTS_SORTED4),   # C3: 74 KB of LDS, two workgroups per CU
    ((20_000, 500, 4096), R.PACK_TREE_LDS),         # C2: N below 32,768 -> whole tree
    ((70_000, 500, 4096), R.PACK_TREE_LDS),         # N < 16 x 2L
    ((200_000, 6, 256), R.PACK_PARTS_SORTED2),
    ((400_000, 500, 2048), R.PACK_PARTS_SORTED2),   # 4-byte staging of 50,000 does not fit
    ((600_000, 4, 16), R.PACK_PARTS_DIRECT),        # parts above 65,535 samples
    ((100_000, 20, 8192), R.PACK_TREE_LDS),         # 16,384 buckets: whole-tree path
    ((100_000, 20, 25_000), R.PACK_TREE_RANGES),
])
def test_pack_plan_paths(args, plan):
    assert R.pack_plan(*args) == plan


def test_pack_plan_rejects_bad_arguments():
    for args in ((0, 5, 5), (10, 0, 5), (10, 5, 0), (10, 5, 5, 0)):
        with pytest.raises(ValueError):
            R.pack_plan(*args)


def test_quant_scale_is_the_reference_rule():
    """rfxp_quant_scale is compute_scale_from_minmax_kernel's float rule
    (cuda/rf_quantization_kernels.cu:88-101): scale = (max - min)/255 in
    float, 1/127 below 1e-10, zp = -min/scale.  Checked against numpy float32
    arithmetic; for min 0, max 1 it gives the C3 parameters fl(1/255), -0."""
    import numpy as np

    f = np.float32
    for mn, mx in ((0.0, 1.0), (0.0125, 1.0), (0.0, 7.5), (-0.25, 0.5), (0.3, 0.3), (1e-12, 2e-12)):
        sc, zp = R.quant_scale(mn, mx)
        want_sc = (f(mx) - f(mn)) / f(255.0)
        if want_sc < f(1e-10):
            want_sc = f(1.0) / f(127.0)
        want_zp = -f(mn) / want_sc
        assert f(sc) == want_sc and f(zp) == want_zp, (mn, mx, sc, zp)
    sc, zp = R.quant_scale(0.0, 1.0)
    assert f(sc) == f(1.0) / f(255.0) and zp == 0.0 and np.signbit(f(zp))
    assert R.quant_scale(0.3, 0.3)[0] == float(f(1.0) / f(127.0))
