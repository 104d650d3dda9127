"""Closed forms that full-size GPU results are checked against (test
infrastructure): quantities the mathematics fixes independently of how the
kernels or the oracle compute them."""
import numpy as np


def pair_total(leaf, oob, nleaf):
    """Sum of U over every pair i < j, from leaf histograms alone: in each
    tree a leaf with o OOB and b in-bag samples contributes o * b pairs
    (each unordered pair of opposite OOB status in one leaf is counted once
    in the upper triangle)."""
    total = 0
    for t in range(leaf.shape[0]):
        lv = leaf[t]
        ok = (lv >= 0) & (lv < nleaf)
        o = np.bincount(lv[ok & (oob[t] != 0)], minlength=nleaf).astype(np.int64)
        b = np.bincount(lv[ok & (oob[t] == 0)], minlength=nleaf).astype(np.int64)
        total += int((o * b).sum())
    return total
