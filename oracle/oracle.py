"""ctypes front end of the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path never does.  It loads ``liboracle.so`` (our
C restatement, built by ``oracle/Makefile``) and, where it was built in the
build container, ``_ref/libref.so`` (the reference's own CPU sources
compiled in place, see ``ref_shim.cpp``).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

FMT_F32, FMT_F16, FMT_I8, FMT_NF4, FMT_U8, FMT_U16 = range(6)
FMT_DTYPE = {FMT_F32: np.float32, FMT_F16: np.uint16, FMT_I8: np.int8,
             FMT_NF4: np.uint8, FMT_U8: np.uint8, FMT_U16: np.uint16}

_P = np.ctypeslib.ndpointer
_i32 = _P(np.int32, flags="C")
_u8 = _P(np.uint8, flags="C")
_u16 = _P(np.uint16, flags="C")
_f64 = _P(np.float64, flags="C")
_f32 = _P(np.float32, flags="C")

_lib = None
_ref = None


def tri_size(n: int) -> int:
    return n * (n + 1) // 2


def tri_idx(n: int, i, j):
    return i * n - i * (i + 1) // 2 + j


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run make -C oracle)")
        L = C.CDLL(path)
        L.orc_cpu_proximity.argtypes = [_i32, _i32, _i32, C.c_int32, C.c_int32, C.c_int, C.c_void_p]
        L.orc_finishprox.argtypes = [C.c_int32, _i32, _f64, _f64]
        L.orc_rfgap.argtypes = [C.c_int32, C.c_int32, _i32, _i32, _f64]
        L.orc_terminal_leaf.argtypes = [_i32, C.c_int32, _i32, C.c_int32, _i32]
        L.orc_p.argtypes = [C.c_uint32, C.c_int32, C.c_int32]
        L.orc_p.restype = C.c_double
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_q_i8.argtypes = [C.c_float, C.c_float, C.c_float]
        L.orc_q_i8.restype = C.c_int8
        L.orc_q_nf4.argtypes = [C.c_float]
        L.orc_q_nf4.restype = C.c_uint8
        L.orc_q_u8.argtypes = [C.c_float, C.c_float, C.c_float]
        L.orc_q_u8.restype = C.c_uint8
        L.orc_u8_scale_from_minmax.argtypes = [C.c_float, C.c_float, C.POINTER(C.c_float),
                                               C.POINTER(C.c_float)]
        L.orc_nout.argtypes = [_u8, C.c_int64, C.c_int32, _i32]
        L.orc_upper_counts_scatter.argtypes = [_i32, _u8, C.c_int64, C.c_int32, C.c_int32, _u16]
        L.orc_upper_rows.argtypes = [_i32, _u8, C.c_int64, C.c_int32, C.c_int32, C.c_void_p,
                                     C.c_int, C.c_float, C.c_float, C.c_int64, C.c_int64,
                                     C.c_void_p, C.c_int]
        L.orc_upper_rows.restype = C.c_int
        L.orc_both_oob_rows.argtypes = [_i32, _u8, C.c_int64, C.c_int32, C.c_int32, C.c_int, C.c_int64,
                                        C.c_int64, C.c_void_p, C.c_int]
        L.orc_both_oob_rows.restype = C.c_int
        L.orc_index_build.argtypes = [_i32, _u8, C.c_int64, C.c_int32, C.c_int32, C.c_void_p, C.c_int]
        L.orc_index_build.restype = C.c_void_p
        L.orc_index_rows.argtypes = [C.c_void_p, C.c_int, C.c_float, C.c_float, C.c_int64, C.c_int64,
                                     C.c_void_p, C.c_int]
        L.orc_index_rows.restype = C.c_int
        L.orc_index_free.argtypes = [C.c_void_p]
        L.orc_upper_from_counts.argtypes = [_u16, _i32, C.c_int64, C.c_int, C.c_float, C.c_float,
                                            C.c_void_p]
        L.orc_topk_all.argtypes = [_i32, C.c_int64, C.c_int32, C.c_int32, _i32, C.c_int64, C.c_int32,
                                   C.c_void_p, _i32, _u16, C.c_int]
        L.orc_topk_oob.argtypes = [_i32, _u8, C.c_int64, C.c_int32, C.c_int32, C.c_int64, C.c_int32, C.c_int,
                                   _i32, _u16, _f32]
        L.orc_topk_oob.restype = C.c_int32
        L.orc_lowrank_pv.argtypes = [_i32, C.c_int64, C.c_int32, C.c_int32, _f64, C.c_int32, _f64]
        L.orc_tree_upper.argtypes = [C.c_int, _i32, _i32, _i32, C.c_int32, C.c_int32, C.c_int, C.c_int32,
                                     C.c_float, C.c_float, C.c_void_p]
        L.orc_rfgap_tree_upper.argtypes = [_i32, _i32, C.c_int32, C.c_int32, C.c_void_p]
        L.orc_dispatch_prox.argtypes = [C.c_int, _i32, _i32, C.c_int32, _i32, _i32, C.c_void_p]
        L.orc_pair_proximity.argtypes = [_i32, _u8, C.c_int64, C.c_int32, C.c_int32, C.c_int64, C.c_int64]
        L.orc_pair_proximity.restype = C.c_float
        L.orc_outlier_raw.argtypes = [_i32, C.c_int64, C.c_int32, C.c_int32, _i32, C.c_int64, C.c_void_p,
                                      C.c_float, C.c_float, _f32, C.c_int]
        L.orc_outlier_normalize.argtypes = [_f32, C.c_int64, C.c_void_p, _f32]
        L.orc_forest_leaves.argtypes = [C.c_int, _i32, _i32, _f32, _i32, C.c_void_p, C.c_void_p, C.c_int32,
                                        C.c_int32, C.c_int32, C.c_int32, _f32, C.c_int64, C.c_void_p, _i32]
        _lib = L
    return _lib


def ref_available() -> bool:
    """Whether the compiled reference was built here (no library is loaded)."""
    return os.path.exists(os.path.join(HERE, "_ref", "libref.so"))


def ref():
    """The compiled reference (build container only); None when absent."""
    global _ref
    if _ref is None:
        path = os.path.join(HERE, "_ref", "libref.so")
        if not os.path.exists(path):
            return None
        R = C.CDLL(path)
        R.ref_set_config.argtypes = [C.c_int, C.c_int, C.c_int]
        R.ref_cpu_proximity.argtypes = [_i32, _i32, _i32, C.c_int32, C.c_int32, _f64]
        R.ref_cpu_finishprox.argtypes = [C.c_int32, _i32, _f64, _f64]
        R.ref_cpu_proximity_rfgap.argtypes = [C.c_int32, C.c_int32, _i32, _i32, _f64]
        _ref = R
    return _ref


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- reference-shaped (column-major N x N double) --------------------------

def cpu_proximity(nodestatus, nodextr, nin, nnode, prox, casewise=False):
    """One tree into ``prox`` (Fortran-ordered N x N float64, accumulated)."""
    n = len(nodextr)
    if not (prox.flags.f_contiguous and prox.dtype == np.float64 and prox.shape == (n, n)):
        raise ValueError("prox must be a Fortran-ordered float64 N x N array")
    lib().orc_cpu_proximity(_c(nodestatus, np.int32), _c(nodextr, np.int32), _c(nin, np.int32),
                            n, nnode, int(casewise), prox.ctypes.data)


def finishprox(nout, prox):
    n = len(nout)
    out = np.zeros((n, n), dtype=np.float64, order="F")
    lib().orc_finishprox(n, _c(nout, np.int32), np.ascontiguousarray(prox.reshape(-1, order="F")),
                         out.reshape(-1, order="F"))
    return out


def rfgap(nin_tn, nodextr_tn):
    t, n = nin_tn.shape
    out = np.zeros((n, n), dtype=np.float64, order="F")
    lib().orc_rfgap(t, n, _c(nin_tn, np.int32).ravel(), _c(nodextr_tn, np.int32).ravel(),
                    out.reshape(-1, order="F"))
    return out


def terminal_leaf(nodestatus, nodextr):
    out = np.empty(len(nodextr), dtype=np.int32)
    lib().orc_terminal_leaf(_c(nodestatus, np.int32), len(nodestatus), _c(nodextr, np.int32),
                            len(nodextr), out)
    return out


# ---- triangle ---------------------------------------------------------------

def nout(oob_tn):
    t, n = oob_tn.shape
    out = np.empty(n, dtype=np.int32)
    lib().orc_nout(_c(oob_tn, np.uint8).ravel(), n, t, out)
    return out


def upper_counts_scatter(leaf_tn, oob_tn, nleaf):
    t, n = leaf_tn.shape
    U = np.empty(tri_size(n), dtype=np.uint16)
    lib().orc_upper_counts_scatter(_c(leaf_tn, np.int32).ravel(), _c(oob_tn, np.uint8).ravel(),
                                   n, t, nleaf, U)
    return U


def out_nbytes(fmt, n_entries):
    if fmt == FMT_NF4:
        return (n_entries + 1) // 2
    return n_entries * np.dtype(FMT_DTYPE[fmt]).itemsize


def both_oob_rows(leaf_tn, oob_tn, nleaf, fmt=FMT_F32, r0=0, r1=None, threads=0):
    """Rows [r0, r1) of the "both OOB" proximity triangle (orc_both_oob_rows):
    F32 P = num / den, or U16 num."""
    t, n = leaf_tn.shape
    r1 = n if r1 is None else r1
    e0, e1 = tri_idx(n, r0, r0), tri_idx(n, r1, r1)
    out = np.zeros(e1 - e0, dtype=np.float32 if fmt == FMT_F32 else np.uint16)
    rc = lib().orc_both_oob_rows(_c(leaf_tn, np.int32).ravel(), _c(oob_tn, np.uint8).ravel(), n, t, nleaf, fmt,
                                 r0, r1, out.ctypes.data, threads)
    assert rc == 0
    return out


def upper_rows(leaf_tn, oob_tn, nleaf, fmt=FMT_U16, scale=1.0, zp=0.0, r0=0, r1=None,
               nout_arr=None, threads=0):
    t, n = leaf_tn.shape
    r1 = n if r1 is None else r1
    e0, e1 = tri_idx(n, r0, r0), tri_idx(n, r1, r1)
    if fmt == FMT_NF4:
        out = np.zeros(((e1 - 1) >> 1) - (e0 >> 1) + 1 if e1 > e0 else 0, dtype=np.uint8)
    else:
        out = np.zeros(e1 - e0, dtype=FMT_DTYPE[fmt])
    na = None
    if nout_arr is not None:
        na = _c(nout_arr, np.int32)
    rc = lib().orc_upper_rows(_c(leaf_tn, np.int32).ravel(), _c(oob_tn, np.uint8).ravel(), n, t,
                              nleaf, na.ctypes.data if na is not None else None, fmt, scale, zp,
                              r0, r1, out.ctypes.data, threads)
    if rc != 0:
        raise ValueError("orc_upper_rows: bad row range")
    return out


class RowIndex:
    """Per-tree buckets built once; rows produced on demand (CPU baseline)."""

    def __init__(self, leaf_tn, oob_tn, nleaf, nout_arr=None, threads=0):
        self.leaf = _c(leaf_tn, np.int32)
        self.oob = _c(oob_tn, np.uint8)
        self.t, self.n = self.leaf.shape
        na = None if nout_arr is None else _c(nout_arr, np.int32)
        self._na = na
        self.h = lib().orc_index_build(self.leaf.ravel(), self.oob.ravel(), self.n, self.t, nleaf,
                                       na.ctypes.data if na is not None else None, threads)

    def rows(self, fmt, r0, r1, scale=1.0, zp=0.0, threads=0):
        n = self.n
        e0, e1 = tri_idx(n, r0, r0), tri_idx(n, r1, r1)
        if fmt == FMT_NF4:
            out = np.zeros(((e1 - 1) >> 1) - (e0 >> 1) + 1 if e1 > e0 else 0, dtype=np.uint8)
        else:
            out = np.zeros(e1 - e0, dtype=FMT_DTYPE[fmt])
        if lib().orc_index_rows(self.h, fmt, scale, zp, r0, r1, out.ctypes.data, threads) != 0:
            raise ValueError("bad row range")
        return out

    def close(self):
        if self.h:
            lib().orc_index_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


def upper_from_counts(U, nout_arr, fmt, scale=1.0, zp=0.0):
    n = len(nout_arr)
    out = np.zeros(out_nbytes(fmt, tri_size(n)) // (1 if fmt == FMT_NF4 else
                                                    np.dtype(FMT_DTYPE[fmt]).itemsize),
                   dtype=FMT_DTYPE[fmt])
    lib().orc_upper_from_counts(_c(U, np.uint16), _c(nout_arr, np.int32), n, fmt, scale, zp,
                                out.ctypes.data)
    return out


def p_value(U, ni, nj):
    return lib().orc_p(U, ni, nj)


def f32_to_f16(x):
    return lib().orc_f32_to_f16(float(x))


def q_i8(v, scale, zp):
    return lib().orc_q_i8(v, scale, zp)


def q_u8(v, scale, zp):
    return lib().orc_q_u8(v, scale, zp)


def q_nf4(v):
    return lib().orc_q_nf4(v)


def u8_scale_from_minmax(vmin, vmax):
    s, z = C.c_float(), C.c_float()
    lib().orc_u8_scale_from_minmax(vmin, vmax, C.byref(s), C.byref(z))
    return s.value, z.value


# ---- top-K ------------------------------------------------------------------

NO_NLEAF = 2**31 - 1   # without nleaf only negative labels are invalid


def topk_all(ref_leaf_tn, qleaf_qt, K, exclude=None, threads=0, nleaf=None):
    """Labels outside [0, nleaf) match nothing (negative ones when nleaf is None)."""
    t, n = ref_leaf_tn.shape
    q = qleaf_qt.shape[0]
    idx = np.empty((q, K), dtype=np.int32)
    cnt = np.empty((q, K), dtype=np.uint16)
    ex = None if exclude is None else _c(exclude, np.int32)
    lib().orc_topk_all(_c(ref_leaf_tn, np.int32).ravel(), n, t, NO_NLEAF if nleaf is None else nleaf,
                       _c(qleaf_qt, np.int32).ravel(), q, K, ex.ctypes.data if ex is not None else None, idx, cnt,
                       threads)
    return idx, cnt


def topk_oob(leaf_tn, oob_tn, q, K, exclude_self=True, nleaf=None):
    t, n = leaf_tn.shape
    idx = np.empty(K, dtype=np.int32)
    cnt = np.empty(K, dtype=np.uint16)
    sc = np.empty(K, dtype=np.float32)
    m = lib().orc_topk_oob(_c(leaf_tn, np.int32).ravel(), _c(oob_tn, np.uint8).ravel(), n, t,
                           NO_NLEAF if nleaf is None else nleaf, q, K, int(exclude_self), idx, cnt, sc)
    return idx[:m], cnt[:m], sc[:m]


# ---- per-tree triangles -------------------------------------------------------

def tree_upper(fmt, nodestatus, nodextr, nin, casewise=False, n_real=0, scale=1.0, zp=0.0):
    """One tree's packed triangle in the reference per-tree formats
    (FMT_F16 -> uint16, FMT_I8 -> int8, FMT_NF4 -> packed uint8)."""
    n = len(nodextr)
    np_ = n_real if 0 < n_real < n else n
    ne = np_ * (np_ + 1) // 2
    out = {FMT_F16: np.zeros(ne, np.uint16), FMT_I8: np.zeros(ne, np.int8),
           FMT_NF4: np.zeros((ne + 1) // 2, np.uint8)}[fmt]
    lib().orc_tree_upper(fmt, _c(nodestatus, np.int32), _c(nodextr, np.int32), _c(nin, np.int32), n,
                         len(nodestatus), int(casewise), n_real, C.c_float(scale), C.c_float(zp),
                         out.ctypes.data)
    return out


def rfgap_tree_upper(nin, nodextr, n_real=0):
    n = len(nin)
    np_ = n_real if 0 < n_real < n else n
    out = np.zeros(np_ * (np_ + 1) // 2, np.uint16)
    lib().orc_rfgap_tree_upper(_c(nin, np.int32), _c(nodextr, np.int32), n, n_real, out.ctypes.data)
    return out


# ---- low rank ---------------------------------------------------------------

def lowrank_pv(leaf_tn, nleaf, V, threads=0):
    """Y = A (A^T V) / T in double (same result for every thread count)."""
    t, n = leaf_tn.shape
    V = _c(V, np.float64)
    r = V.shape[1]
    Y = np.empty_like(V)
    lib().orc_lowrank_pv(_c(leaf_tn, np.int32).ravel(), n, t, nleaf, V.ravel(), r, Y.ravel(), threads)
    return Y


# ---- quantization dispatcher --------------------------------------------------

DISPATCH_DTYPE = {0: np.float64, 1: np.uint16, 2: np.int8, 3: np.uint8}


def dispatch_prox(level, nodexb, nin, ndbegin, npcase):
    """One launch of QuantizationDispatcher::launch_proximity_kernel at
    ``level`` into a zeroed column-major N x N array of that level's type."""
    n = len(nodexb)
    out = np.zeros(n * n, dtype=DISPATCH_DTYPE[level])
    lib().orc_dispatch_prox(level, _c(nodexb, np.int32), _c(nin, np.int32), n, _c(ndbegin, np.int32),
                            _c(npcase, np.int32), out.ctypes.data)
    return out.reshape((n, n), order="F")


# ---- pair proximity and outlier scores ------------------------------------------

def pair_proximity(leaf_tn, oob_tn, nleaf, i, j):
    t, n = leaf_tn.shape
    return lib().orc_pair_proximity(_c(leaf_tn, np.int32).ravel(), _c(oob_tn, np.uint8).ravel(), n, t, nleaf,
                                    int(i), int(j))


def outlier_raw(ref_leaf_tn, nleaf, qleaf_qt, exclude=None, numerator=1.0, isolated=1e10, threads=0):
    t, n = ref_leaf_tn.shape
    q = qleaf_qt.shape[0]
    out = np.empty(q, np.float32)
    ex = None if exclude is None else _c(exclude, np.int32)
    lib().orc_outlier_raw(_c(ref_leaf_tn, np.int32).ravel(), n, t, nleaf, _c(qleaf_qt, np.int32).ravel(), q,
                          ex.ctypes.data if ex is not None else None, numerator, isolated, out, threads)
    return out


def outlier_normalize(raw, classes=None):
    raw = _c(raw, np.float32)
    out = np.empty_like(raw)
    cl = None if classes is None else _c(classes, np.int32)
    lib().orc_outlier_normalize(raw, len(raw), cl.ctypes.data if cl is not None else None, out)
    return out


# ---- leaf assignments on a forest ---------------------------------------------

def forest_leaves(mode, forest, X, nin=None):
    """forest: dict of nodestatus, bestvar, xbestsplit (T x maxnode), treemap
    (T x maxnode x 2), catgoleft (T x maxnode x maxcat) or None, cat (mdim)
    or None.  Returns leaf (T x N) int32."""
    ns = _c(forest["nodestatus"], np.int32)
    t, maxnode = ns.shape
    X = _c(X, np.float32)
    n, mdim = X.shape
    cg = forest.get("catgoleft")
    maxcat = 1 if cg is None else cg.shape[2]
    cg = None if cg is None else _c(cg, np.int32)
    cat = forest.get("cat")
    cat = None if cat is None else _c(cat, np.int32)
    ni = None if nin is None else _c(nin, np.int32)
    out = np.empty((t, n), np.int32)
    lib().orc_forest_leaves(mode, ns.ravel(), _c(forest["bestvar"], np.int32).ravel(),
                            _c(forest["xbestsplit"], np.float32).ravel(), _c(forest["treemap"], np.int32).ravel(),
                            None if cg is None else cg.ctypes.data, None if cat is None else cat.ctypes.data, t,
                            maxnode, maxcat, mdim, X.ravel(), n, None if ni is None else ni.ctypes.data, out.ravel())
    return out
