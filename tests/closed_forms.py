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


def row_pair_counts(leaf, oob, nleaf):
    """Per sample i, the sum over j != i of U_ij (both halves of the
    symmetric matrix): in each tree where i's leaf is valid, U gains 1 for
    every sample of i's leaf with the other OOB bit, so the sum is the size
    of that opposite bucket summed over the trees."""
    ntree, n = leaf.shape
    out = np.zeros(n, dtype=np.int64)
    for t in range(ntree):
        lv = leaf[t].astype(np.int64)
        ok = (lv >= 0) & (lv < nleaf)
        key = np.where(ok, 2 * lv + (oob[t] != 0), 0)
        cnt = np.bincount(key[ok], minlength=2 * nleaf)
        out += np.where(ok, cnt[key ^ 1], 0)
    return out
