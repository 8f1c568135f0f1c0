"""Children with rows but no hessian, quantized gradients, on a real MI355X.

With min_sum_hessian_in_leaf = 0 and lambda_l2 = 0, a split that isolates rows whose
hessians all quantize to 0 has an enormous gain, so the learner takes it.  The smaller
child then has rows but a sum_hessian <= 0, and its f64 cells are cleared before the
subtraction (learner.rs:4061-4089 scans a leaf only with rows and hessian): the
reference's larger sibling is the parent's cells, not its own integers.  The device
keeps such a larger child, and every larger child below it, in its f64 slot instead
of deriving its cells from integers; the trees must still equal the oracle's bit for
bit, on the record and on the wide layout.  Each case checks that its data really
produces such a split.
"""
import os

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend
from lightgbm_rs_amd.synth import config1_like
from oracle import oracle
from tests.datagen import binary_gh

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint64 if a.dtype == np.float64 else np.uint32)


def backend(records):
    """A context created with LGBM_HIP_RECORDS=`records` (read at creation)."""
    old = os.environ.get("LGBM_HIP_RECORDS")
    if records is None:
        os.environ.pop("LGBM_HIP_RECORDS", None)
    else:
        os.environ["LGBM_HIP_RECORDS"] = records
    try:
        return HipBackend(0)
    finally:
        if old is None:
            os.environ.pop("LGBM_HIP_RECORDS", None)
        else:
            os.environ["LGBM_HIP_RECORDS"] = old


def zero_hessian_smaller_children(o):
    """Leaves with rows, sum_hessian <= 0 and fewer rows than their sibling."""
    lw, lc, lp = (np.asarray(o[k]) for k in ("leaf_weight", "leaf_count", "leaf_parent"))
    lch, rch, ic = (np.asarray(o[k]) for k in ("left_child", "right_child", "internal_count"))
    hits = []
    for leaf in range(o["num_leaves"]):
        if lc[leaf] > 0 and lw[leaf] <= 0.0:
            p = lp[leaf]
            sib = rch[p] if lch[p] == ~leaf else lch[p]
            sc = lc[~sib] if sib < 0 else ic[sib]
            if lc[leaf] < sc:
                hits.append(leaf)
    return hits


@pytest.mark.parametrize("records,n,nl,seed", [
    (None, 60_000, 63, 1),
    ("wide", 60_000, 63, 2),
    (None, 300_000, 255, 3),
    ("wide", 300_000, 255, 4),
])
def test_zero_hessian_smaller_child_matches_oracle(records, n, nl, seed):
    say(f"zero-hessian children records={records} n={n} num_leaves={nl} seed={seed}")
    bins, meta, ub, _ = config1_like(n, seed=seed)
    g, h, _ = binary_gh(n, seed=seed)
    h = h.copy()
    h[bins[3] <= 2] = 1e-7  # quantizes to 0 (scale = max h / 4)
    cfg = GainConfig.make(min_data_in_leaf=1, min_sum_hessian_in_leaf=0.0, lambda_l2=0.0)
    og, oh, _, _ = oracle.quantize(g, h, bins=4, stochastic=True, seed=seed * 77)
    o, olay = oracle.train_tree(bins, meta, ub, og, oh, cfg, nl, -1)
    assert zero_hessian_smaller_children(o), "the data must produce a zeroed smaller child"
    be = backend(records)
    try:
        be.upload_resident_bins(bins, meta, ub)
        be.upload_resident_grad_hess(g, h)
        _, dg, dh = be.discretize_dequantize_in_place(4, True, seed * 77, want_values=True)
        assert np.array_equal(bits(dg), bits(og)) and np.array_equal(bits(dh), bits(oh))
        t, lay = be.grow_tree_on_device_with_cfg(cfg, nl, -1)
    finally:
        be.close()
    assert t["num_leaves"] == o["num_leaves"]
    for k in o:
        if k == "num_leaves":
            continue
        a, b = np.asarray(t[k]), np.asarray(o[k])
        if a.dtype.kind == "f":
            assert np.array_equal(bits(a), bits(b)), k
        else:
            assert np.array_equal(a, b), k
    assert np.array_equal(lay["leaf_count"], olay["leaf_count"])
