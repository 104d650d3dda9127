#!/usr/bin/env python3
"""Writes the golden fixtures of this directory from the reference's OWN CPU
proximity code, compiled in place from /root/reference by oracle/Makefile
into oracle/_ref/libref.so (build container only; the GPU box has neither
the reference tree nor this step).  Only inputs and outputs are stored.

Fixtures
  cpu_prox_small.npz  random trees (terminal and non-terminal nodes, node
                      indices out of range, bootstrap multiplicities, rows
                      with nout = 0): rf::cpu_proximity accumulated over the
                      trees (casewise off and on) and rf::cpu_finishprox.
  c1_forest.npz       the first benchmark configuration (N=2000, p=20, T=100, mtry=4,
                      nodesize=1): leaf matrix of a CART forest grown here on
                      seeded bootstraps, plus SHA-256 digests of the
                      reference's packed count triangle, of (float)P of its
                      finishprox output, and of the uint8 codes of (float)P
                      (scale=1/255, zp=0) computed with numpy; and 20,000
                      sampled entries.
  rfgap_small.npz     rf::cpu_proximity_rfgap on random trees.

Usage: python tests/golden/make_golden.py   (after `make -C oracle`)
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
import oracle as O  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def ref_forest(R, nodestatus, nodextr, nin, nnode_per_tree, casewise):
    t, n = nodextr.shape
    R.ref_set_config(int(casewise), 0, 4)
    prox = np.zeros((n, n), order="F")
    for k in range(t):
        R.ref_cpu_proximity(np.ascontiguousarray(nodestatus[k, :nnode_per_tree[k]], dtype=np.int32),
                            np.ascontiguousarray(nodextr[k], dtype=np.int32),
                            np.ascontiguousarray(nin[k], dtype=np.int32), n, int(nnode_per_tree[k]),
                            prox.reshape(-1, order="F"))
    return prox


def ref_finish(R, nout, prox):
    n = len(nout)
    out = np.zeros((n, n), order="F")
    R.ref_cpu_finishprox(n, np.ascontiguousarray(nout, dtype=np.int32),
                         np.ascontiguousarray(prox.reshape(-1, order="F")), out.reshape(-1, order="F"))
    return out


def small_random(R):
    rng = np.random.default_rng(20261201)
    n, t, nnode = 120, 40, 31
    nodestatus = np.where(rng.random((t, nnode)) < 0.7, -1, rng.integers(1, 3, (t, nnode))).astype(np.int8)
    nodextr = rng.integers(-2, nnode + 2, (t, n)).astype(np.int16)
    nin = np.zeros((t, n), dtype=np.uint8)
    for k in range(t):
        nin[k] = np.bincount(rng.integers(0, n, n), minlength=n)
    nin[:, :3] = 1  # rows 0..2 never OOB: nout = 0
    nnodes = np.full(t, nnode)
    nout = (nin == 0).sum(axis=0).astype(np.int32)
    out = dict(nodestatus=nodestatus, nodextr=nodextr, nin=nin, nout=nout)
    for cw in (0, 1):
        prox = ref_forest(R, nodestatus.astype(np.int32), nodextr.astype(np.int32), nin.astype(np.int32),
                          nnodes, cw)
        out[f"prox_cw{cw}"] = prox
        out[f"proxsym_cw{cw}"] = ref_finish(R, nout, prox)
    np.savez_compressed(os.path.join(HERE, "cpu_prox_small.npz"), **out)


def c1_forest(R):
    from sklearn.tree import DecisionTreeClassifier

    seed = 20261201 + 1
    rng = np.random.default_rng(seed)
    n, p, t = 2000, 20, 100
    X = rng.standard_normal((n, p)).astype(np.float32)
    y = (X[:, 0] + 0.5 * X[:, 1] + rng.normal(0, 0.3, n) > 0).astype(np.int32)
    leaf = np.zeros((t, n), dtype=np.int32)
    nin = np.zeros((t, n), dtype=np.uint8)
    nodestatus = []
    nnodes = np.zeros(t, dtype=np.int32)
    for k in range(t):
        boot = rng.integers(0, n, n)
        nin[k] = np.bincount(boot, minlength=n)
        clf = DecisionTreeClassifier(max_features=4, min_samples_leaf=1,
                                     random_state=int(rng.integers(0, 2**31 - 1)))
        clf.fit(X[boot], y[boot])
        leaf[k] = clf.apply(X)
        st = np.where(clf.tree_.children_left == -1, -1, 1).astype(np.int32)
        nodestatus.append(st)
        nnodes[k] = len(st)
    ns = np.full((t, nnodes.max()), 2, dtype=np.int32)
    for k in range(t):
        ns[k, :nnodes[k]] = nodestatus[k]
    nout = (nin == 0).sum(axis=0).astype(np.int32)
    prox = ref_forest(R, ns, leaf, nin.astype(np.int32), nnodes, 0)
    proxsym = ref_finish(R, nout, prox)
    iu = np.triu_indices(n)
    full = prox + prox.T
    U = full[iu]
    U[iu[0] == iu[1]] = 0
    assert np.all(U == np.round(U)) and U.max() < 65536
    U16 = U.astype(np.uint16)
    P32 = proxsym[iu].astype(np.float32)
    scale = np.float32(1.0) / np.float32(255.0)
    r = P32 / scale + np.float32(0.0)
    codes = np.clip(r, np.float32(0), np.float32(255)).astype(np.uint8)
    samp = np.random.default_rng(5).integers(0, len(U16), 20000)
    # terminal ordinals per tree (what the batched path takes as leaf labels)
    lab = np.zeros_like(leaf)
    for k in range(t):
        lab[k] = O.terminal_leaf(ns[k, :nnodes[k]], leaf[k])
    nleaf = int(lab.max()) + 1
    np.savez_compressed(
        os.path.join(HERE, "c1_forest.npz"),
        node=leaf.astype(np.int16), nodestatus=ns.astype(np.int8), nnodes=nnodes, nin=nin,
        label=lab.astype(np.int16), nleaf=nleaf, nout=nout,
        sha_u16=sha(U16), sha_p32=sha(P32), sha_u8=sha(codes),
        samp_idx=samp, samp_u=U16[samp], samp_p=proxsym[iu][samp], u_max=int(U16.max()),
        zero_pairs=int((U16 == 0).sum() - n))


def rfgap_small(R):
    rng = np.random.default_rng(20261201 + 10)
    n, t, nnode = 80, 30, 15
    nodextr = rng.integers(-1, nnode, (t, n)).astype(np.int32)
    nin = np.zeros((t, n), dtype=np.int32)
    for k in range(t):
        nin[k] = np.bincount(rng.integers(0, n, n), minlength=n)
    nin[:, 0] = 1  # sample 0 never OOB: diagonal rule
    R.ref_set_config(0, 0, 2)
    out = np.zeros((n, n), order="F")
    R.ref_cpu_proximity_rfgap(t, n, np.ascontiguousarray(nin.ravel()), np.ascontiguousarray(nodextr.ravel()),
                              out.reshape(-1, order="F"))
    np.savez_compressed(os.path.join(HERE, "rfgap_small.npz"), nin=nin.astype(np.uint8),
                        nodextr=nodextr.astype(np.int8), prox=out)


def main():
    R = O.ref()
    if R is None:
        sys.exit("oracle/_ref/libref.so is not built (needs /root/reference and `make -C oracle`)")
    small_random(R)
    c1_forest(R)
    rfgap_small(R)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
