"""Python front end of librfxprox.so (the MI355X proximity library).

A thin ctypes layer over the C ABI declared in include/rfx_prox.h.  Device
buffers are torch tensors on a HIP device; torch is only the allocator and
stream provider here, every kernel comes from librfxprox.so.  There is no
CPU fallback: if the library is missing or no GPU is visible, calls raise.

The reference exposes this path through C++ (rf::cpu_proximity /
rf::cpu_finishprox, include/rf_proximity.hpp:10-14, include/rf_finishprox.hpp:9;
rf::cuda::gpu_proximity_upper_triangle*, include/rf_proximity_upper_triangle.hpp:42-156),
which the same library implements with those signatures; this module is the
batched interface used by the tests and the benchmark.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "librfxprox.so")
REPO = os.path.dirname(HERE)
HEADER = os.path.join(REPO, "include", "rfx_prox.h")

LEAVES_PREDICT, LEAVES_TRAIN = 0, 1
FMT_F32, FMT_F16, FMT_I8, FMT_NF4, FMT_U8, FMT_U16 = range(6)
FMT_NAMES = {"f32": FMT_F32, "f16": FMT_F16, "i8": FMT_I8, "nf4": FMT_NF4, "u8": FMT_U8,
             "u16": FMT_U16}

_lib = None


class RfxpError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"rfxp error {code}: {msg}")
        self.code = code


def header_functions(path: str = HEADER):
    """Names of the functions declared in the C header."""
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(rfxp_\w+)\s*\(", src, flags=re.M)


def load(path: str = LIB_PATH):
    """Loads librfxprox.so; raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"librfxprox.so not built at {path}: run `make -C rfx-fuse_amd`")
    L = C.CDLL(path)
    vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int32
    L.rfxp_ctx_create.argtypes = [C.c_int, C.POINTER(vp)]
    L.rfxp_ctx_destroy.argtypes = [vp]
    L.rfxp_ctx_set_stream.argtypes = [vp, vp]
    L.rfxp_ctx_stream.argtypes = [vp]
    L.rfxp_ctx_stream.restype = vp
    L.rfxp_ctx_own_stream.argtypes = [vp]
    L.rfxp_ctx_own_stream.restype = vp
    L.rfxp_sync.argtypes = [vp]
    L.rfxp_last_error.argtypes = [vp, C.c_char_p, C.c_size_t]
    L.rfxp_set_timing.argtypes = [vp, C.c_int]
    L.rfxp_kernel_time.argtypes = [vp, C.c_char_p, C.POINTER(C.c_double), C.POINTER(i64)]
    L.rfxp_reset_timing.argtypes = [vp]
    L.rfxp_set_forest.argtypes = [vp, vp, i64, i64, vp, i64, i64, i32, i32, vp]
    L.rfxp_upper.argtypes = [vp, C.c_int, C.c_float, C.c_float, i64, i64, vp]
    L.rfxp_upper_nbytes.argtypes = [C.c_int, i64, i64, i64]
    L.rfxp_upper_nbytes.restype = i64
    L.rfxp_get_nout.argtypes = [vp, vp]
    L.rfxp_upper_minmax.argtypes = [vp, i64, i64, vp]
    L.rfxp_quant_scale.argtypes = [C.c_float, C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]
    L.rfxp_quant_scale.restype = None
    L.rfxp_upper_recounts.argtypes = [vp, C.POINTER(i64)]
    L.rfxp_upper_work_item.argtypes = [i64, i32, i64, i64, i64, C.POINTER(i64), C.POINTER(i64)]
    L.rfxp_upper_work_item.restype = i64
    L.rfxp_upper_launches.argtypes = [i64]
    L.rfxp_upper_launches.restype = i64
    L.rfxp_pack_plan.argtypes = [i64, i32, i32, i32]
    L.rfxp_pack_plan.restype = C.c_int
    L.rfxp_upper_noalloc.argtypes = [vp, vp, i64, i64, vp, i64, i64, i32, i32, vp, C.c_int, C.c_float, C.c_float,
                                     i64, i64, vp]
    L.rfxp_both_oob.argtypes = [vp, vp, i64, i64, vp, i64, i64, i32, i32, C.c_int, i64, i64, vp]
    L.rfxp_upper_noalloc_workspace.argtypes = [i64, i32, i32, C.c_int]
    L.rfxp_upper_noalloc_workspace.restype = i64
    L.rfxp_set_reference.argtypes = [vp, vp, i64, i64, i64, i32, i32]
    L.rfxp_topk.argtypes = [vp, vp, i64, i64, i64, vp, i64, i64, i32, C.c_int, vp, vp]
    L.rfxp_topk_scores.argtypes = [vp, vp, i64, i64, i32, i32, vp, vp, vp]
    L.rfxp_pair_proximity.argtypes = [vp, vp, i64, i64, vp, i64, i64, i32, i32, vp, vp, i64, vp]
    L.rfxp_outlier_raw.argtypes = [vp, vp, i64, i64, i64, i64, vp, C.c_float, C.c_float, vp]
    L.rfxp_outlier_normalize.argtypes = [vp, i64, vp, vp, vp, vp]
    L.rfxp_forest_leaves.argtypes = [vp, C.c_int, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i64, vp, C.c_int,
                                     vp, vp, i64]
    L.rfxp_symacc_reset.argtypes = [vp, i64]
    L.rfxp_symacc_nnz.argtypes = [vp]
    L.rfxp_symacc_nnz.restype = i64
    L.rfxp_symacc_device_bytes.argtypes = [vp]
    L.rfxp_symacc_device_bytes.restype = i64
    L.rfxp_symacc_add_upper.argtypes = [vp, C.c_int, vp, C.c_float, C.c_float]
    L.rfxp_symacc_add_dense.argtypes = [vp, vp]
    L.rfxp_symacc_apply.argtypes = [vp, vp, i32, vp]
    L.rfxp_symacc_factor.argtypes = [vp, i32, i32, C.c_uint64, vp, vp]
    L.rfxp_factor_reconstruct.argtypes = [vp, vp, vp, i64, i32, vp, vp]
    L.rfxp_factor_mds.argtypes = [vp, vp, i64, i32, i32, vp, i32, vp, vp]
    L.rfxp_factor_quantized_bytes.argtypes = [C.c_int, i64]
    L.rfxp_factor_quantized_bytes.restype = i64
    L.rfxp_factor_quantize.argtypes = [vp, C.c_int, vp, i64, vp, vp]
    L.rfxp_factor_dequantize.argtypes = [vp, C.c_int, vp, i64, vp, vp]
    L.rfxp_host_symeig.argtypes = [i32, vp, vp, vp]
    L.rfxp_lowrank_pv.argtypes = [vp, vp, i32, vp]
    L.rfxp_lowrank_oob_pv.argtypes = [vp, vp, i32, vp]
    L.rfxp_lowrank_subspace.argtypes = [vp, vp, i32, i32, vp, vp]
    L.rfxp_tree_pairs.argtypes = [vp, vp, vp, vp, i32, i32, C.c_int, C.POINTER(C.POINTER(i64)),
                                  C.POINTER(C.POINTER(C.c_double)), C.POINTER(i64)]
    L.rfxp_tree_accumulate.argtypes = [vp, vp, vp, vp, i32, i32, C.c_int, vp]
    L.rfxp_tree_upper.argtypes = [vp, C.c_int, vp, vp, vp, i32, i32, C.c_int, i32, C.c_float, C.c_float, vp]
    L.rfxp_rfgap_tree_upper.argtypes = [vp, vp, vp, i32, i32, vp]
    L.rfxp_finishprox.argtypes = [vp, i32, vp, vp, vp]
    L.rfxp_rfgap.argtypes = [vp, i32, i32, vp, vp, vp]
    _lib = L
    return L


def upper_nbytes(fmt: int, n: int, r0: int = 0, r1: int | None = None) -> int:
    r1 = n if r1 is None else r1
    v = load().rfxp_upper_nbytes(fmt, n, r0, r1)
    if v < 0:
        raise ValueError("bad format or row range")
    return v


PACK_PARTS_DIRECT, PACK_PARTS_SORTED2, PACK_PARTS_SORTED4, PACK_TREE_LDS, PACK_TREE_RANGES = range(5)
GFX950_MAX_LDS = 163840


def pack_plan(n: int, t: int, nleaf: int, max_lds: int = GFX950_MAX_LDS) -> int:
    """Packing path rfxp_set_forest takes for a forest of this shape
    (PACK_* codes; host only)."""
    v = load().rfxp_pack_plan(n, t, nleaf, max_lds)
    if v < 0:
        raise ValueError("bad arguments")
    return v


def upper_work_items(n: int, s: int, r0: int, r1: int):
    """Segments (row, first column) of rfxp_upper's decomposition of rows
    [r0, r1) into S-column segments, in launch order (host only)."""
    L = load()
    cnt = L.rfxp_upper_work_item(n, s, r0, r1, -1, None, None)
    if cnt < 0:
        raise ValueError("bad arguments")
    out = []
    row, col = C.c_int64(), C.c_int64()
    for e in range(cnt):
        L.rfxp_upper_work_item(n, s, r0, r1, e, C.byref(row), C.byref(col))
        out.append((row.value, col.value))
    return out


def upper_noalloc_workspace(n: int, t: int, nleaf: int, nout_given: bool = False) -> int:
    """Device workspace bytes rfxp_upper_noalloc needs for a forest."""
    return load().rfxp_upper_noalloc_workspace(n, t, nleaf, int(nout_given))


NOALLOC_MAX_BYTES = 64 << 20


def quant_scale(min_val: float, max_val: float):
    """(scale, zero_point) of the reference's affine quantizer rule for a
    min and max (rfxp_quant_scale, host only)."""
    sc, zp = C.c_float(), C.c_float()
    load().rfxp_quant_scale(min_val, max_val, C.byref(sc), C.byref(zp))
    return sc.value, zp.value


def outlier_normalize(raw, classes=None):
    """Host: (scores, medians, mads) of rfxp_outlier_normalize (numpy in/out)."""
    import numpy as np

    L = load()
    raw = np.ascontiguousarray(raw, dtype=np.float32)
    n = raw.shape[0]
    cls = None if classes is None else np.ascontiguousarray(classes, dtype=np.int32)
    ng = 1 if cls is None else len(np.unique(cls))
    sc = np.empty(n, np.float32)
    med = np.empty(ng, np.float32)
    mad = np.empty(ng, np.float32)
    rc = L.rfxp_outlier_normalize(raw.ctypes.data, n, None if cls is None else cls.ctypes.data, sc.ctypes.data,
                                  med.ctypes.data, mad.ctypes.data)
    if rc != 0:
        raise RfxpError(rc, "rfxp_outlier_normalize: bad arguments")
    return sc, med, mad


def pack_oob_bits(oob_tn):
    """(T, N) bool/uint8 torch tensor -> (T, ceil(N/32)) int32 words, bit i%32
    of word i//32 set when sample i is OOB."""
    import torch

    t, n = oob_tn.shape
    w = (n + 31) // 32
    pad = torch.zeros((t, w * 32), dtype=torch.int64, device=oob_tn.device)
    pad[:, :n] = oob_tn.to(torch.int64)
    weights = (torch.ones(32, dtype=torch.int64, device=oob_tn.device) << torch.arange(
        32, device=oob_tn.device))
    words = (pad.view(t, w, 32) * weights).sum(dim=2)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words)
    return words.to(torch.int32).contiguous()


class Context:
    """One librfxprox context (device, stream, resident forest index)."""

    def __init__(self, device: int = 0):
        self._L = load()
        h = C.c_void_p()
        rc = self._L.rfxp_ctx_create(device, C.byref(h))
        if rc != 0:
            buf = C.create_string_buffer(512)
            self._L.rfxp_last_error(None, buf, 512)
            raise RfxpError(rc, buf.value.decode())
        self.h = h
        self.device = device

    def close(self):
        if getattr(self, "h", None):
            self._L.rfxp_ctx_destroy(self.h)
            self.h = None
        self._forest_inputs = None
        self._reference_leaf = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc != 0:
            buf = C.create_string_buffer(1024)
            self._L.rfxp_last_error(self.h, buf, 1024)
            raise RfxpError(rc, buf.value.decode())

    def set_stream(self, stream_handle: int | None):
        self._check(self._L.rfxp_ctx_set_stream(self.h, stream_handle))

    def use_torch_stream(self):
        import torch

        self.set_stream(torch.cuda.current_stream(self.device).cuda_stream)

    def sync(self):
        self._check(self._L.rfxp_sync(self.h))

    def set_timing(self, on: bool):
        self._check(self._L.rfxp_set_timing(self.h, int(on)))

    def kernel_time(self, name: str):
        ms, n = C.c_double(), C.c_int64()
        self._check(self._L.rfxp_kernel_time(self.h, name.encode(), C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def reset_timing(self):
        self._check(self._L.rfxp_reset_timing(self.h))

    def set_forest(self, leaf, oob_words, n: int, t: int, nleaf: int, layout: str = "tree",
                   nout=None):
        """leaf: int32 device tensor, (T, N) for layout 'tree' or (N, T) for
        'sample'; oob_words: int32 device tensor (T, ceil(N/32))."""
        import torch

        assert leaf.dtype == torch.int32 and leaf.is_cuda and leaf.is_contiguous()
        assert oob_words.dtype == torch.int32 and oob_words.is_cuda and oob_words.is_contiguous()
        if layout == "tree":
            si, st = 1, n
        elif layout == "sample":
            si, st = t, 1
        else:
            raise ValueError(layout)
        nptr = None
        if nout is not None:
            assert nout.dtype == torch.int32 and nout.is_cuda
            nptr = nout.data_ptr()
        self._check(self._L.rfxp_set_forest(self.h, leaf.data_ptr(), si, st, oob_words.data_ptr(),
                                            oob_words.shape[1], n, t, nleaf, nptr))
        # rfxp_lowrank_oob_pv reads these later: keep them alive with the forest
        self._forest_inputs = (leaf, oob_words)
        self.n = n
        self.t = t

    def set_reference(self, leaf, n: int, t: int, nleaf: int, layout: str = "tree"):
        """Reference set for top-K: leaf int32 device tensor, (T, N) for
        layout 'tree' or (N, T) for 'sample'."""
        import torch

        assert leaf.dtype == torch.int32 and leaf.is_cuda and leaf.is_contiguous()
        si, st = (1, n) if layout == "tree" else (t, 1)
        self._check(self._L.rfxp_set_reference(self.h, leaf.data_ptr(), si, st, n, t, nleaf))
        # rfxp_lowrank_pv reads the leaf matrix later: keep it alive with the set
        self._reference_leaf = leaf
        self.ref_n = n

    def topk(self, qleaf, k: int, layout: str = "sample", oob_words=None, exclude_base: int = -1,
             positive_only: bool = False):
        """Top-k references per query: qleaf int32 device tensor, (Q, T) for
        layout 'sample' or (T, Q) for 'tree'; oob_words (T, ceil(Q/32))
        int32 device tensor restricting each query to its OOB trees.
        Returns (idx int32 (Q, k), counts int16-viewed-uint16 (Q, k))."""
        import torch

        assert qleaf.dtype == torch.int32 and qleaf.is_cuda and qleaf.is_contiguous()
        if layout == "sample":
            q, t = qleaf.shape
            si, st = t, 1
        else:
            t, q = qleaf.shape
            si, st = 1, q
        idx = torch.empty((q, k), dtype=torch.int32, device=qleaf.device)
        cnt = torch.empty((q, k), dtype=torch.int16, device=qleaf.device)
        optr, old = None, 0
        if oob_words is not None:
            assert oob_words.dtype == torch.int32 and oob_words.is_cuda and oob_words.is_contiguous()
            optr, old = oob_words.data_ptr(), oob_words.shape[1]
        self._check(self._L.rfxp_topk(self.h, qleaf.data_ptr(), si, st, q, optr, old, exclude_base, k,
                                      int(positive_only), idx.data_ptr(), cnt.data_ptr()))
        return idx, cnt

    def topk_scores(self, idx, cnt, t: int, oob_words=None):
        """Float scores of topk results (OOB queries when oob_words is the
        topk call's OOB words, else new queries over t trees)."""
        import torch

        q, k = idx.shape
        sc = torch.empty((q, k), dtype=torch.float32, device=idx.device)
        optr, old = None, 0
        if oob_words is not None:
            optr, old = oob_words.data_ptr(), oob_words.shape[1]
        self._check(self._L.rfxp_topk_scores(self.h, optr, old, q, t, k, idx.data_ptr(), cnt.data_ptr(),
                                             sc.data_ptr()))
        return sc

    def pair_proximity(self, leaf, oob_words, n: int, t: int, nleaf: int, pi, pj, layout: str = "tree"):
        """compute_proximity_from_leaves for pairs (pi[p], pj[p]) (int64
        device tensors); leaf int32 (T, N) for layout 'tree' or (N, T)."""
        import torch

        assert leaf.dtype == torch.int32 and leaf.is_cuda and leaf.is_contiguous()
        si, st = (1, n) if layout == "tree" else (t, 1)
        assert pi.dtype == torch.int64 and pj.dtype == torch.int64 and pi.shape == pj.shape
        out = torch.empty(pi.shape[0], dtype=torch.float32, device=leaf.device)
        self._check(self._L.rfxp_pair_proximity(self.h, leaf.data_ptr(), si, st, oob_words.data_ptr(),
                                                oob_words.shape[1], n, t, nleaf, pi.data_ptr(), pj.data_ptr(),
                                                pi.shape[0], out.data_ptr()))
        return out

    def outlier_raw(self, qleaf, layout: str = "sample", exclude_base: int = -1, exclude_idx=None,
                    numerator: float = 1.0, isolated: float = 1e10):
        """Raw outlier measure of each query against the reference set."""
        import torch

        assert qleaf.dtype == torch.int32 and qleaf.is_cuda and qleaf.is_contiguous()
        if layout == "sample":
            q, t = qleaf.shape
            si, st = t, 1
        else:
            t, q = qleaf.shape
            si, st = 1, q
        raw = torch.empty(q, dtype=torch.float32, device=qleaf.device)
        ex = None if exclude_idx is None else exclude_idx.data_ptr()
        self._check(self._L.rfxp_outlier_raw(self.h, qleaf.data_ptr(), si, st, q, exclude_base, ex,
                                             numerator, isolated, raw.data_ptr()))
        return raw

    def forest_leaves(self, mode: int, forest: dict, X, nin=None, terminal_only: bool = False, oob: bool = False):
        """forest: dict of device tensors nodestatus, bestvar (int32), xbestsplit
        (float32) (T, maxnode), treemap (T, maxnode, 2), optional catgoleft
        (T, maxnode, maxcat) and cat (mdim,); X (N, mdim) float32 device.
        Returns leaf (T, N) int32 and, with oob=True (training mode), the
        OOB words (T, ceil(N/32)) int32."""
        import torch

        ns = forest["nodestatus"]
        t, maxnode = ns.shape
        n, mdim = X.shape
        cg, cat = forest.get("catgoleft"), forest.get("cat")
        maxcat = 1 if cg is None else cg.shape[2]
        leaf = torch.empty((t, n), dtype=torch.int32, device=X.device)
        words = torch.empty((t, (n + 31) // 32), dtype=torch.int32, device=X.device) if oob else None
        self._check(self._L.rfxp_forest_leaves(
            self.h, mode, ns.data_ptr(), forest["bestvar"].data_ptr(), forest["xbestsplit"].data_ptr(),
            forest["treemap"].data_ptr(), None if cg is None else cg.data_ptr(),
            None if cat is None else cat.data_ptr(), t, maxnode, maxcat, mdim, X.data_ptr(), n,
            None if nin is None else nin.data_ptr(), int(terminal_only), leaf.data_ptr(),
            None if words is None else words.data_ptr(), 0 if words is None else words.shape[1]))
        return (leaf, words) if oob else leaf

    # ---- accumulated symmetric matrix and its factor (low-rank class engine)

    def symacc_reset(self, n: int):
        self._check(self._L.rfxp_symacc_reset(self.h, n))

    def symacc_nnz(self) -> int:
        return self._L.rfxp_symacc_nnz(self.h)

    def symacc_device_bytes(self) -> int:
        return self._L.rfxp_symacc_device_bytes(self.h)

    def symacc_add_upper(self, fmt: int, tri, scale: float = 1.0, zp: float = 0.0):
        """tri: a device tensor or a host numpy array (packed triangle)."""
        ptr = tri.data_ptr() if hasattr(tri, "data_ptr") else tri.ctypes.data
        self._check(self._L.rfxp_symacc_add_upper(self.h, fmt, ptr, scale, zp))

    def symacc_add_dense(self, full):
        ptr = full.data_ptr() if hasattr(full, "data_ptr") else full.ctypes.data
        self._check(self._L.rfxp_symacc_add_dense(self.h, ptr))

    def symacc_apply(self, X):
        import torch

        assert X.dtype == torch.float64 and X.is_cuda and X.is_contiguous()
        Y = torch.empty_like(X)
        self._check(self._L.rfxp_symacc_apply(self.h, X.data_ptr(), X.shape[1], Y.data_ptr()))
        return Y

    def symacc_factor(self, n: int, rank: int, iters: int, seed: int = 1):
        """(A device (rank, n) tensor holding the column-major N x rank factor, Ritz values)."""
        import numpy as np
        import torch

        A = torch.empty((rank, n), dtype=torch.float64, device="cuda:0")
        ev = np.empty(rank)
        self._check(self._L.rfxp_symacc_factor(self.h, rank, iters, seed, A.data_ptr(), ev.ctypes.data))
        return A, ev

    def factor_reconstruct(self, A_cm, n: int, rank: int, oob_counts=None):
        """A_cm: device (rank, n) float64 (column-major N x rank); returns the
        device (n, n) tensor holding the column-major reconstruction."""
        import numpy as np
        import torch

        out = torch.empty((n, n), dtype=torch.float64, device="cuda:0")
        cnt = None if oob_counts is None else np.ascontiguousarray(oob_counts, dtype=np.int32)
        self._check(self._L.rfxp_factor_reconstruct(self.h, A_cm.data_ptr(), A_cm.data_ptr(), n, rank,
                                                    None if cnt is None else cnt.ctypes.data, out.data_ptr()))
        return out

    def factor_mds(self, A_cm, n: int, rank: int, k: int, oob_counts=None, iters: int = 100):
        import numpy as np

        cnt = None if oob_counts is None else np.ascontiguousarray(oob_counts, dtype=np.int32)
        coords = np.empty((n, k))
        ev = np.empty(k)
        self._check(self._L.rfxp_factor_mds(self.h, A_cm.data_ptr(), n, rank, k,
                                            None if cnt is None else cnt.ctypes.data, iters, coords.ctypes.data,
                                            ev.ctypes.data))
        return coords, ev

    def factor_quantize(self, level: int, A, scale_zp=None):
        import torch

        nb = self._L.rfxp_factor_quantized_bytes(level, A.numel())
        q = torch.empty(max(nb, 1), dtype=torch.uint8, device=A.device)
        self._check(self._L.rfxp_factor_quantize(self.h, level, A.data_ptr(), A.numel(),
                                                 None if scale_zp is None else scale_zp.data_ptr(), q.data_ptr()))
        return q

    def factor_dequantize(self, level: int, q, count: int, scale_zp=None):
        import torch

        A = torch.empty(count, dtype=torch.float64, device=q.device)
        self._check(self._L.rfxp_factor_dequantize(self.h, level, q.data_ptr(), count,
                                                   None if scale_zp is None else scale_zp.data_ptr(), A.data_ptr()))
        return A

    def lowrank_oob_pv(self, V):
        """Y = P V for the OOB-normalised proximity of the current forest."""
        import torch

        assert V.dtype == torch.float32 and V.is_cuda and V.is_contiguous()
        Y = torch.empty_like(V)
        self._check(self._L.rfxp_lowrank_oob_pv(self.h, V.data_ptr(), V.shape[1], Y.data_ptr()))
        return Y

    def lowrank_pv(self, V):
        """Y = P V for the reference set (P = A A^T / T): V float32 device
        tensor (N, r), r <= 64."""
        import torch

        assert V.dtype == torch.float32 and V.is_cuda and V.is_contiguous() and V.dim() == 2
        Y = torch.empty_like(V)
        self._check(self._L.rfxp_lowrank_pv(self.h, V.data_ptr(), V.shape[1], Y.data_ptr()))
        return Y

    def lowrank_subspace(self, V0, iters: int):
        """Rank-r factor (Q, B) of P by subspace iteration; V0 float32 device
        (N, r), r <= 32.  Returns Q (device, N x r) and B (numpy r x r)."""
        import numpy as np
        import torch

        assert V0.dtype == torch.float32 and V0.is_cuda and V0.is_contiguous() and V0.dim() == 2
        r = V0.shape[1]
        Q = torch.empty_like(V0)
        B = np.zeros((r, r), dtype=np.float64)
        self._check(self._L.rfxp_lowrank_subspace(self.h, V0.data_ptr(), r, iters, Q.data_ptr(),
                                                  B.ctypes.data))
        return Q, B

    def upper(self, fmt: int, out, r0: int = 0, r1: int | None = None, scale: float = 1.0,
              zp: float = 0.0):
        r1 = self.n if r1 is None else r1
        need = upper_nbytes(fmt, self.n, r0, r1)
        have = out.numel() * out.element_size()
        if have < need:
            raise ValueError(f"output buffer has {have} bytes, rows need {need}")
        self._check(self._L.rfxp_upper(self.h, fmt, scale, zp, r0, r1, out.data_ptr()))
        return out

    def both_oob(self, leaf, oob_words, n: int, t: int, nleaf: int, fmt: int = 0, r0: int = 0,
                 r1: int | None = None, layout: str = "tree"):
        """rfxp_both_oob: rows [r0, r1) of the both-OOB proximity triangle,
        F32 (num / den) or U16 (num), as a new device tensor."""
        import torch

        assert leaf.dtype == torch.int32 and leaf.is_cuda and leaf.is_contiguous()
        assert oob_words.dtype == torch.int32 and oob_words.is_cuda and oob_words.is_contiguous()
        si, st = (1, n) if layout == "tree" else (t, 1)
        r1 = n if r1 is None else r1
        # a bad range is left for the library to reject
        ne = upper_nbytes(FMT_U16, n, r0, r1) // 2 if 0 <= r0 <= r1 <= n else 1
        out = torch.empty(max(ne, 1), dtype=torch.float32 if fmt == FMT_F32 else torch.int16, device=leaf.device)
        self._check(self._L.rfxp_both_oob(self.h, leaf.data_ptr(), si, st, oob_words.data_ptr(), oob_words.shape[1],
                                          n, t, nleaf, fmt, r0, r1, out.data_ptr()))
        return out[:ne]

    def upper_noalloc(self, leaf, oob_words, n: int, t: int, nleaf: int, fmt: int, out, r0: int = 0,
                      r1: int | None = None, scale: float = 1.0, zp: float = 0.0, layout: str = "tree",
                      nout=None):
        """rfxp_upper_noalloc: set_forest + upper in one call, with the forest
        index in the library's static device workspace (no allocation)."""
        import torch

        assert leaf.dtype == torch.int32 and leaf.is_cuda and leaf.is_contiguous()
        assert oob_words.dtype == torch.int32 and oob_words.is_cuda and oob_words.is_contiguous()
        si, st = (1, n) if layout == "tree" else (t, 1)
        r1 = n if r1 is None else r1
        need = upper_nbytes(fmt, n, r0, r1)
        have = out.numel() * out.element_size()
        if have < need:
            raise ValueError(f"output buffer has {have} bytes, rows need {need}")
        nptr = None if nout is None else nout.data_ptr()
        self._check(self._L.rfxp_upper_noalloc(self.h, leaf.data_ptr(), si, st, oob_words.data_ptr(),
                                               oob_words.shape[1], n, t, nleaf, nptr, fmt, scale, zp, r0, r1,
                                               out.data_ptr()))
        return out

    def upper_minmax(self, r0: int = 0, r1: int | None = None):
        """(min, max) of the fp32 entries of rows [r0, r1) of the triangle
        (rfxp_upper_minmax): the data of the reference's quantizer rule."""
        import numpy as np

        r1 = self.n if r1 is None else r1
        mm = np.zeros(2, dtype=np.float32)
        self._check(self._L.rfxp_upper_minmax(self.h, r0, r1, mm.ctypes.data))
        return float(mm[0]), float(mm[1])

    def upper_recounts(self) -> int:
        """Row segments recounted with 16-bit counters since set_forest."""
        v = C.c_int64()
        self._check(self._L.rfxp_upper_recounts(self.h, C.byref(v)))
        return v.value

    def nout(self):
        import torch

        out = torch.empty(self.n, dtype=torch.int32, device=f"cuda:{self.device}")
        self._check(self._L.rfxp_get_nout(self.h, out.data_ptr()))
        return out

    # ---- per-tree and dense small-N operations (host numpy arrays) ----------

    @staticmethod
    def _i32(a):
        import numpy as np

        return np.ascontiguousarray(a, dtype=np.int32)

    def tree_pairs(self, nodestatus, nodextr, nin, casewise: bool = False):
        """OOB x in-bag pairs of one tree: (idx int64, w float64) numpy copies."""
        import numpy as np

        ns, nx, ni = self._i32(nodestatus), self._i32(nodextr), self._i32(nin)
        pi, pw, cnt = C.POINTER(C.c_int64)(), C.POINTER(C.c_double)(), C.c_int64()
        self._check(self._L.rfxp_tree_pairs(self.h, ns.ctypes.data, nx.ctypes.data, ni.ctypes.data, len(nx),
                                            len(ns), int(casewise), C.byref(pi), C.byref(pw), C.byref(cnt)))
        n = cnt.value
        if n == 0:
            return np.zeros(0, np.int64), np.zeros(0, np.float64)
        return (np.ctypeslib.as_array(pi, (n,)).copy(), np.ctypeslib.as_array(pw, (n,)).copy())

    def tree_accumulate(self, nodestatus, nodextr, nin, prox, casewise: bool = False):
        """One tree into prox (Fortran-ordered N x N float64 numpy, in place)."""
        import numpy as np

        ns, nx, ni = self._i32(nodestatus), self._i32(nodextr), self._i32(nin)
        n = len(nx)
        assert prox.dtype == np.float64 and prox.shape == (n, n) and prox.flags.f_contiguous
        self._check(self._L.rfxp_tree_accumulate(self.h, ns.ctypes.data, nx.ctypes.data, ni.ctypes.data, n,
                                                 len(ns), int(casewise), prox.ctypes.data))
        return prox

    def tree_upper(self, fmt: int, nodestatus, nodextr, nin, casewise: bool = False, n_real: int = 0,
                   scale: float = 1.0, zp: float = 0.0):
        """One tree's packed triangle (host numpy: uint16 for F16, int8 for
        I8, packed uint8 for NF4)."""
        import numpy as np

        ns, nx, ni = self._i32(nodestatus), self._i32(nodextr), self._i32(nin)
        n = len(nx)
        m = n_real if 0 < n_real < n else n
        ne = m * (m + 1) // 2
        out = {FMT_F16: lambda: np.zeros(ne, np.uint16), FMT_I8: lambda: np.zeros(ne, np.int8),
               FMT_NF4: lambda: np.zeros((ne + 1) // 2, np.uint8)}.get(fmt, lambda: np.zeros(2 * ne, np.uint8))()
        self._check(self._L.rfxp_tree_upper(self.h, fmt, ns.ctypes.data, nx.ctypes.data, ni.ctypes.data, n,
                                            len(ns), int(casewise), n_real, scale, zp, out.ctypes.data))
        return out

    def tree_upper_device(self, fmt: int, nodestatus, nodextr, nin, out, casewise: bool = False,
                          n_real: int = 0, scale: float = 1.0, zp: float = 0.0):
        """rfxp_tree_upper into a device tensor `out` (4-byte aligned, byte
        size a multiple of 4)."""
        ns, nx, ni = self._i32(nodestatus), self._i32(nodextr), self._i32(nin)
        self._check(self._L.rfxp_tree_upper(self.h, fmt, ns.ctypes.data, nx.ctypes.data, ni.ctypes.data,
                                            len(nx), len(ns), int(casewise), n_real, scale, zp, out.data_ptr()))
        return out

    def rfgap_tree_upper(self, nin, nodextr, n_real: int = 0):
        import numpy as np

        ni, nx = self._i32(nin), self._i32(nodextr)
        n = len(ni)
        m = n_real if 0 < n_real < n else n
        out = np.zeros(m * (m + 1) // 2, np.uint16)
        self._check(self._L.rfxp_rfgap_tree_upper(self.h, ni.ctypes.data, nx.ctypes.data, n, n_real,
                                                  out.ctypes.data))
        return out

    def finishprox(self, nout, prox):
        """Dense symmetrised, nout-normalised proximity (Fortran N x N)."""
        import numpy as np

        no = self._i32(nout)
        n = len(no)
        src = np.asfortranarray(prox, dtype=np.float64)
        out = np.zeros((n, n), np.float64, order="F")
        self._check(self._L.rfxp_finishprox(self.h, n, no.ctypes.data, src.ctypes.data, out.ctypes.data))
        return out

    def rfgap(self, nin_tn, nodextr_tn):
        """RF-GAP proximity of T trees, (T, N) inputs, Fortran N x N output."""
        import numpy as np

        ni, nx = self._i32(nin_tn), self._i32(nodextr_tn)
        t, n = ni.shape
        out = np.zeros((n, n), np.float64, order="F")
        self._check(self._L.rfxp_rfgap(self.h, t, n, ni.ctypes.data, nx.ctypes.data, out.ctypes.data))
        return out
