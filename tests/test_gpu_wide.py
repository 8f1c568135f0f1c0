"""The wide row layout (REC_FMT_WIDE: bins in a fixed row-major matrix, the partition
moving row indices) on the device against the oracle and against the record layouts.

  * forced onto configs[1]'s shape (LGBM_HIP_RECORDS=wide): quantized boosting bit-exact
    with the oracle and with the packed-record layout; f32-gradient boosting bit-exact
    with the record layout (64-bit fixed-point cells are exact integers, so the layout
    cannot change a bit) and structurally identical to the oracle;
  * F = 300 (beyond the records' 124): quantized boosting, trees and scores bit-exact,
    and the layout export (partition order) equal to DataPartition::split's;
  * configs[2]'s shape (2000 sparse LogNormal columns, 90% zeros, f32 gradients) and
    configs[4]'s shape (700 U(0,1) columns with 30% zeros, quantized) at reduced rows;
  * configs[3]'s mix (numerical and categorical columns, softmax multiclass) forced
    onto the wide layout: the categorical scan and the bitset routing of the 1-byte
    wide layout, trees and scores bit-exact with the oracle;
  * device binning of a wide raw table (lgbm_hip_upload_raw) against the host mappers.
The most frequent bin of every feature is never accumulated in this layout
(FixHistogram rebuilds it, compaction drops it); these trees pin that it changes
nothing the scans see.
"""
import os

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend
from lightgbm_rs_amd.synth import (config1_like, config2_binned, config3_binned,
                                   config4_binned, _bin_columns)
from oracle import oracle

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def bits(a):
    return np.ascontiguousarray(a, np.float64).view(np.uint64)


def _mrz(v):
    z = float(np.float32(1e-35))
    return np.where((v >= -z) & (v <= z), 0.0, v)


def backend(records=None):
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


STRUCT = ("split_feature", "threshold_in_bin", "decision_type", "left_child", "right_child",
          "leaf_count", "internal_count", "leaf_depth", "leaf_parent")
VALUES = ("threshold", "leaf_value", "internal_value", "internal_weight", "leaf_weight")


def train(bins, meta, ub, y, nl, iters, qbins, records=None, cfg=None):
    """Binary boosting on the device: (trees, scores, init score)."""
    init = oracle.boost_from_score(y)
    cfg = cfg or GainConfig.make(min_data_in_leaf=20)
    b = backend(records)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.set_labels(y, init)
        trees = [b.train_iter_binary(i, cfg, nl, -1, 0.1, qbins, True) for i in range(iters)]
        scores = b.scores()
    finally:
        b.close()
    return trees, scores, init


def assert_same_trees(ta, tb, tag):
    assert len(ta) == len(tb), tag
    for i, (a, b) in enumerate(zip(ta, tb)):
        assert a["num_leaves"] == b["num_leaves"], (tag, i)
        for k in STRUCT + VALUES + ("split_gain",):
            assert np.array_equal(np.asarray(a[k]).view(np.uint8), np.asarray(b[k]).view(np.uint8)), (tag, i, k)


def assert_matches_oracle(trees, scores, otrees, oscores, init, tag, exact=True):
    assert len(trees) == len(otrees), tag
    for i, (t, o) in enumerate(zip(trees, otrees)):
        t = dict(t)
        if i == 0 and init != 0.0:
            t["leaf_value"] = _mrz(t["leaf_value"] + init)
            t["internal_value"] = _mrz(t["internal_value"] + init)
        assert t["num_leaves"] == o["num_leaves"], (tag, i)
        for k in STRUCT:
            assert np.array_equal(np.asarray(t[k]), np.asarray(o[k])), (tag, i, k)
        for k in VALUES:
            a, b = np.asarray(t[k], np.float64), np.asarray(o[k], np.float64)
            if exact:
                assert np.array_equal(bits(a), bits(b)), (tag, i, k)
            else:
                np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-300, err_msg=f"{tag} {i} {k}")
    if exact:
        assert np.array_equal(bits(scores), bits(oscores)), tag
    else:
        np.testing.assert_allclose(scores, oscores, rtol=1e-9, atol=1e-12, err_msg=tag)


def test_wide_forced_config1_shape_quantized():
    n, iters, nl = 120_000, 3, 63
    say(f"wide forced, configs[1] shape n={n}, quantized")
    bins, meta, ub, y = config1_like(n, seed=21)
    tw, sw, init = train(bins, meta, ub, y, nl, iters, 4, records="wide")
    tp, sp, _ = train(bins, meta, ub, y, nl, iters, 4)
    assert_same_trees(tw, tp, "wide vs packed records")
    assert np.array_equal(bits(sw), bits(sp))
    oscores, otrees = oracle.train_binary(bins, meta, ub, y, GainConfig.make(min_data_in_leaf=20),
                                          nl, -1, iters, 0.1)
    assert_matches_oracle(tw, sw, otrees, oscores, init, "wide vs oracle")


def test_wide_forced_config1_shape_f32():
    n, iters, nl = 120_000, 3, 63
    say(f"wide forced, configs[1] shape n={n}, f32 gradients")
    bins, meta, ub, y = config1_like(n, seed=22, max_bin=255)
    tw, sw, init = train(bins, meta, ub, y, nl, iters, 0, records="wide")
    tr, sr, _ = train(bins, meta, ub, y, nl, iters, 0, records="legacy")
    assert_same_trees(tw, tr, "wide vs legacy records (fixed point)")
    assert np.array_equal(bits(sw), bits(sr))
    oscores, otrees = oracle.train_binary(bins, meta, ub, y, GainConfig.make(min_data_in_leaf=20),
                                          nl, -1, iters, 0.1, quantized=False)
    assert_matches_oracle(tw, sw, otrees, oscores, init, "wide f32 vs oracle", exact=False)


def _wide_data(n, F, seed, max_bin=255):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((F, n)).astype(np.float32)
    X[rng.random((F, n)) < 0.2] = 0.0
    w = rng.standard_normal(F) / np.sqrt(F)
    logit = X.astype(np.float64).T @ w * 3.0 + 0.5 * X[0] * X[1]
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-logit))).astype(np.float32)
    bins, meta, ub, ms = _bin_columns(X, max_bin)
    return X, y, bins, meta, ub, ms


def test_wide_300_features_quantized_and_layout():
    n, F, iters, nl = 60_000, 300, 3, 63
    say(f"wide F={F} n={n} quantized")
    X, y, bins, meta, ub, ms = _wide_data(n, F, 31)
    assert sum(m.num_bin for m in meta) > 8192
    trees, scores, init = train(bins, meta, ub, y, nl, iters, 4)
    cfg = GainConfig.make(min_data_in_leaf=20)
    oscores, otrees = oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, iters, 0.1)
    assert_matches_oracle(trees, scores, otrees, oscores, init, "F=300 quantized")
    # one tree from given gradients with its partition layout (f32 gradients)
    rng = np.random.default_rng(5)
    g = rng.standard_normal(n).astype(np.float32)
    h = rng.uniform(0.05, 0.25, n).astype(np.float32)
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.upload_resident_grad_hess(g, h)
        t, lay = b.grow_tree_on_device_with_cfg(cfg, 127, -1)
    finally:
        b.close()
    o, olay = oracle.train_tree(bins, meta, ub, g, h, cfg, 127, -1)
    assert t["num_leaves"] == o["num_leaves"]
    for k in STRUCT:
        assert np.array_equal(t[k], o[k]), k
    for k in ("leaf_value", "internal_value", "leaf_weight", "threshold"):
        np.testing.assert_allclose(t[k], o[k], rtol=1e-9, atol=1e-12, err_msg=k)
    assert np.array_equal(lay["indices"], olay["indices"])
    assert np.array_equal(lay["leaf_begin"], olay["leaf_begin"])


def test_wide_config2_shape_f32():
    n, F, iters, nl = 40_000, 2000, 2, 127
    say(f"configs[2] shape n={n} F={F} f32 gradients")
    bins, meta, ub, t = config2_binned(n, F=F)
    y = (t > np.median(t)).astype(np.float32)
    trees, scores, init = train(bins, meta, ub, y, nl, iters, 0)
    cfg = GainConfig.make(min_data_in_leaf=20)
    oscores, otrees = oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, iters, 0.1,
                                          quantized=False)
    assert_matches_oracle(trees, scores, otrees, oscores, init, "configs[2] shape", exact=False)


def test_wide_config4_shape_quantized():
    n, F, iters, nl = 60_000, 700, 2, 255
    say(f"configs[4] shape n={n} F={F} quantized")
    bins, meta, ub, rel, _ = config4_binned(n, F=F)
    y = (rel >= 3).astype(np.float32)
    trees, scores, init = train(bins, meta, ub, y, nl, iters, 4)
    cfg = GainConfig.make(min_data_in_leaf=20)
    oscores, otrees = oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, iters, 0.1)
    assert_matches_oracle(trees, scores, otrees, oscores, init, "configs[4] shape")


def test_wide_device_binning_matches_mappers():
    n, F = 30_000, 260
    say(f"wide device binning n={n} F={F}")
    X, y, bins, meta, ub, ms = _wide_data(n, F, 41)
    X[3, ::7] = np.nan
    bins[3] = ms[3].value_to_bin(X[3]).astype(np.uint8)
    for col_major in (True, False):
        b = HipBackend(0)
        try:
            src = X if col_major else np.ascontiguousarray(X.T)
            b.upload_raw(src, ms, col_major=col_major)
            got = b.get_bins()
        finally:
            b.close()
        assert np.array_equal(got, bins), col_major


def test_wide_forced_categorical_multiclass_matches_oracle():
    n, K, nl, iters = 60_000, 10, 31, 2
    bins, meta, vals, y, cat, _, _ = config3_binned(n, seed=0x5EED0063)
    assert cat, "the data must hold categorical columns"
    cfg = GainConfig.make(min_data_in_leaf=20)
    prior = np.bincount(y.astype(np.int64), minlength=K) / n
    init = np.log(np.maximum(prior, 1e-15))
    applied = np.where(np.abs(init) > 1e-15, init, 0.0)
    say(f"wide categorical multiclass n={n} K={K}")
    b = backend("wide")
    try:
        b.upload_resident_bins(bins, meta, vals)
        b.set_labels_multiclass(y, K, applied)
        trees = []
        for it in range(iters):
            for k, t in enumerate(b.train_iter_multiclass(it, cfg, nl, -1, 0.1, 4, True, [1] * K)):
                t = dict(t)
                if it == 0 and abs(init[k]) > 1e-15:
                    t["leaf_value"] = _mrz(t["leaf_value"] + init[k])
                    t["internal_value"] = _mrz(t["internal_value"] + init[k])
                trees.append(t)
        scores = b.scores()
    finally:
        b.close()
    oscores, otrees = oracle.train_multiclass(bins, meta, vals, y, K, cfg, nl, -1, iters, 0.1,
                                              quantized=True, quant_bins=4, stochastic=True)
    assert len(trees) == len(otrees) == K * iters
    assert any(int(t["num_cat"]) > 0 for t in trees), "no categorical split was exercised"
    for i, (t, o) in enumerate(zip(trees, otrees)):
        assert t["num_leaves"] == o["num_leaves"], i
        for k in o:
            if k == "num_leaves":
                continue
            a, c = np.ascontiguousarray(t[k]), np.ascontiguousarray(o[k])
            assert a.shape == c.shape and a.tobytes() == c.tobytes(), (i, k)
    assert np.array_equal(bits(scores), bits(oscores))


def _train_env(env, bins, meta, ub, y, nl, iters, qbins):
    """train() with extra environment switches read at context creation."""
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return train(bins, meta, ub, y, nl, iters, qbins)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("qbins", [4, 0])
def test_wide_without_feature_major_copy_matches(qbins):
    """The wide layout routes partitions (and builds an f32 root histogram) from its
    feature-major copy of the bins when that copy fits; without it (LGBM_HIP_BINCOL=0,
    as when the allocation fails) the router reads the row's binmat byte.  Both give
    the same trees and scores, bit for bit."""
    n, F, iters, nl = 50_000, 300, 2, 63
    say(f"wide F={F} n={n} qbins={qbins} with and without the feature-major copy")
    X, y, bins, meta, ub, ms = _wide_data(n, F, 37)
    ta, sa, _ = train(bins, meta, ub, y, nl, iters, qbins)
    tb, sb, _ = _train_env({"LGBM_HIP_BINCOL": "0"}, bins, meta, ub, y, nl, iters, qbins)
    assert_same_trees(ta, tb, "bincol vs binmat router")
    assert np.array_equal(bits(sa), bits(sb))
