"""L2 regression, LambdaRank and per-tree column sampling on the device (configs[2]
and configs[4]'s paths) against the oracle and the real binary's captures.

  * LambdaRank gradients on the device bit-exact with the real binary's iteration-1
    capture and with the oracle at trained scores (configs[4]'s query shape);
  * the real binary's 10-iteration lambdarank model (f32 gradients): trees and raw
    scores;
  * the real binary's feature_fraction cells (binary objective, f32 gradients): each
    tree's split features and the raw predictions;
  * configs[2]'s workload at reduced rows (2000 sparse columns, L2, f32 gradients,
    feature_fraction 0.8, 127 leaves) and configs[4]'s (700 columns, lambdarank over
    Poisson(120) queries, quantized, 255 leaves) against the oracle's boosting loop:
    structure exact; quantized leaf values and scores bit-exact, f32 ones within
    1e-9 relative (64-bit fixed-point histograms vs the f64 fold; the stated f32 bar
    is 1e-5).
"""
import json
import os

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend, boost_from_score, feature_mappers, feature_meta
from lightgbm_rs_amd.synth import config2_binned, config4_binned
from oracle import oracle

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def say(*a):
    print(*a, flush=True)


def bits(a):
    return np.ascontiguousarray(a, np.float64).view(np.uint64)


def _mrz(v):
    z = float(np.float32(1e-35))
    return np.where((v >= -z) & (v <= z), 0.0, v)


STRUCT = ("split_feature", "threshold_in_bin", "decision_type", "left_child", "right_child",
          "leaf_count", "internal_count")
VALUES = ("threshold", "leaf_value", "internal_value", "internal_weight", "leaf_weight")


def compare(trees, scores, otrees, oscores, init, tag, exact):
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
        if exact:  # every other field of the tree too
            for k in o:
                if k in STRUCT or k in VALUES or k == "num_leaves":
                    continue
                a, b = np.ascontiguousarray(t[k]), np.ascontiguousarray(o[k])
                assert a.shape == b.shape and a.tobytes() == b.tobytes(), (tag, i, k)
    if exact:
        assert np.array_equal(bits(scores), bits(oscores)), tag
    else:
        np.testing.assert_allclose(scores, oscores, rtol=1e-9, atol=1e-12, err_msg=tag)


def device_boost(bins, meta, ub, y, objective, nl, iters, qbins, feature_fraction=1.0,
                 query_boundaries=None, rank_kw=None, cfg=None):
    init = boost_from_score(objective, y)
    cfg = cfg or GainConfig.make(min_data_in_leaf=20)
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.set_labels(y, init if abs(init) > float(np.float32(1e-15)) else 0.0)
        if objective == "lambdarank":
            b.set_lambdarank(query_boundaries, **(rank_kw or {}))
        else:
            b.set_objective(objective)
        if feature_fraction < 1.0:
            b.set_col_sampler(feature_fraction, 1.0, 2)
        trees = []
        for i in range(iters):
            t = b.train_iter(i, cfg, nl, -1, 0.1, qbins, True)
            trees.append(t)
            if t["num_leaves"] <= 1:
                break
        scores = b.scores()
        g, h = b.gradients()
    finally:
        b.close()
    return trees, scores, init, (g, h)


# --- LambdaRank ----------------------------------------------------------------------
def _rank():
    with open(os.path.join(GOLD, "lambdarank.json")) as f:
        return json.load(f)


def _rank_inputs(d):
    X = np.array(d["X"], dtype=np.float64)
    y = np.array(d["label_bits"], dtype=np.uint32).view(np.float32)
    qb = np.array(d["query_boundaries"], dtype=np.int32)
    ms = feature_mappers(X, max_bin=255, min_data_in_bin=1, min_data_in_leaf=1)
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    return X, y, qb, bins, meta, ub


def test_lambdarank_real_binary_on_device():
    d = _rank()
    X, y, qb, bins, meta, ub = _rank_inputs(d)
    say("lambdarank corpus on device")
    cfg = GainConfig.make(min_data_in_leaf=1, min_sum_hessian_in_leaf=1e-3)
    kw = dict(sigmoid=d["sigmoid"], norm=d["lambdarank_norm"], truncation_level=d["truncation_level"])
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.set_labels(y, 0.0)
        b.set_lambdarank(qb, **kw)
        trees = []
        for i in range(d["num_iterations"]):
            trees.append(b.train_iter(i, cfg, d["num_leaves"], -1, d["learning_rate"], 0, True))
            if i == 0:  # the gradients at zero scores: the real binary's iteration 1
                g, h = b.gradients()
                assert g.view(np.uint32).tolist() == d["gh_iter1"]["GRAD"]
                assert h.view(np.uint32).tolist() == d["gh_iter1"]["HESS"]
        scores = b.scores()
    finally:
        b.close()
    for i, (t, gt) in enumerate(zip(trees, d["trees"])):
        nl = int(gt["num_leaves"][0])
        assert t["num_leaves"] == nl, i
        assert t["split_feature"][:nl - 1].tolist() == [int(v) for v in gt["split_feature"]], i
        assert t["leaf_count"][:nl].tolist() == [int(v) for v in gt["leaf_count"]], i
        lv = np.array([float(v) for v in gt["leaf_value"]])  # shrunk, as the model stores them
        np.testing.assert_allclose(t["leaf_value"][:nl], lv, rtol=1e-9, atol=1e-15, err_msg=str(i))
    want = np.array(d["score_bits"], dtype=np.uint64).view(np.float64)
    np.testing.assert_allclose(scores, want, rtol=1e-9, atol=1e-12)


def test_lambdarank_gradients_match_oracle_at_trained_scores():
    n, F = 30_000, 40
    bins, meta, ub, rel, groups = config4_binned(n, F=F, seed=0x5EED0044)
    qb = np.concatenate([[0], np.cumsum(groups)]).astype(np.int32)
    say(f"lambdarank gradients n={n} queries={len(groups)}")
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.set_labels(rel, 0.0)
        b.set_lambdarank(qb)
        cfg = GainConfig.make(min_data_in_leaf=20)
        for i in range(3):
            b.train_iter(i, cfg, 63, -1, 0.1, 4, True)
        s = b.scores()
        b.train_iter(3, cfg, 63, -1, 0.1, 4, True)  # evaluates the gradients at s
        g, h = b.gradients()
    finally:
        b.close()
    og, oh = oracle.lambdarank_gradients(s, rel, qb)
    assert np.array_equal(g.view(np.uint32), og.view(np.uint32))
    assert np.array_equal(h.view(np.uint32), oh.view(np.uint32))


def test_config4_shape_lambdarank_quantized():
    n, F, iters, nl = 60_000, 700, 2, 255
    bins, meta, ub, rel, groups = config4_binned(n, F=F)
    qb = np.concatenate([[0], np.cumsum(groups)]).astype(np.int32)
    say(f"configs[4] shape n={n} F={F} queries={len(groups)} lambdarank quantized")
    trees, scores, init, _ = device_boost(bins, meta, ub, rel, "lambdarank", nl, iters, 4,
                                          query_boundaries=qb)
    cfg = GainConfig.make(min_data_in_leaf=20)
    oscores, otrees = oracle.train(bins, meta, ub, rel, cfg, oracle.OBJECTIVE_LAMBDARANK, nl, -1,
                                   iters, 0.1, quantized=True, query_boundaries=qb)
    compare(trees, scores, otrees, oscores, 0.0, "configs[4] shape", exact=True)


# --- L2 regression, column sampling --------------------------------------------------
def test_config2_shape_l2_feature_fraction():
    n, F, iters, nl = 40_000, 2000, 3, 127
    bins, meta, ub, y = config2_binned(n, F=F)
    say(f"configs[2] shape n={n} F={F} L2 feature_fraction 0.8")
    trees, scores, init, _ = device_boost(bins, meta, ub, y, "regression", nl, iters, 0,
                                          feature_fraction=0.8)
    cfg = GainConfig.make(min_data_in_leaf=20)
    oscores, otrees = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_REGRESSION, nl, -1,
                                   iters, 0.1, quantized=False, feature_fraction=0.8,
                                   feature_fraction_seed=2)
    compare(trees, scores, otrees, oscores, init, "configs[2] shape", exact=False)


def test_l2_quantized_matches_oracle():
    n, F, iters, nl = 80_000, 30, 3, 63
    rng = np.random.default_rng(17)
    X = rng.standard_normal((F, n)).astype(np.float32)
    y = (X[0] * 2.0 - X[1] + 0.5 * X[2] * X[3] + rng.normal(0, 0.3, n)).astype(np.float32)
    ms = feature_mappers(X.T.astype(np.float64), max_bin=63, min_data_in_leaf=20)
    bins = np.stack([m.value_to_bin(X[j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    say(f"L2 quantized n={n} F={F} feature_fraction 0.5")
    trees, scores, init, _ = device_boost(bins, meta, ub, y, "regression", nl, iters, 4,
                                          feature_fraction=0.5)
    cfg = GainConfig.make(min_data_in_leaf=20)
    oscores, otrees = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_REGRESSION, nl, -1,
                                   iters, 0.1, quantized=True, feature_fraction=0.5,
                                   feature_fraction_seed=2)
    compare(trees, scores, otrees, oscores, init, "L2 quantized", exact=True)


@pytest.mark.parametrize("cell", [0, 1, 2, 3])
def test_feature_fraction_real_binary_on_device(cell):
    z = np.load(os.path.join(GOLD, "feature_fraction.npz"))
    X, y = z["X"], z["y"].astype(np.float32)
    ms = feature_mappers(X, max_bin=63, min_data_in_leaf=5)
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    ff = float(z["fractions"][cell])
    off = int(z["split_counts"][:cell].sum())
    want = []
    for c in z["split_counts"][cell]:
        want.append(sorted(z["split_flat"][off:off + c].tolist()))
        off += c
    say(f"feature_fraction {ff} on device")
    cfg = GainConfig.make(min_data_in_leaf=5)
    trees, scores, init, _ = device_boost(bins, meta, ub, y, "binary", 8, int(z["num_iterations"]),
                                          0, feature_fraction=ff, cfg=cfg)
    for t, w in zip(trees, want):
        assert sorted(set(int(v) for v in t["split_feature"][:t["num_leaves"] - 1])) == w
    np.testing.assert_allclose(scores, z["pred_bits"][cell].view(np.float64), rtol=1e-9, atol=1e-12)


# --- configs[2] and configs[4] at their full sizes ------------------------------------
def _full_chain(X, ms, y, objective, nl, qbins, feature_fraction=1.0, qb=None, iters=1):
    """The library's own chain: device binning of the raw table (lgbm_hip_upload_raw,
    wide layout) -> `iters` resident boosting iterations; returns the device's bins
    too."""
    init = boost_from_score(objective, y)
    cfg = GainConfig.make(min_data_in_leaf=20)
    b = HipBackend(0)
    try:
        b.upload_raw(X, ms, col_major=True)
        bins = b.get_bins()
        b.set_labels(y, init if abs(init) > float(np.float32(1e-15)) else 0.0)
        if objective == "lambdarank":
            b.set_lambdarank(qb)
        else:
            b.set_objective(objective)
        if feature_fraction < 1.0:
            b.set_col_sampler(feature_fraction, 1.0, 2)
        trees = [b.train_iter(i, cfg, nl, -1, 0.1, qbins, True) for i in range(iters)]
        scores = b.scores()
    finally:
        b.close()
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    return trees, scores, init, bins, meta, ub, cfg


def test_config2_full_size():
    """1,000,000 x 2,000 (90% zeros, LogNormal nonzeros), L2, f32
    gradients, feature_fraction 0.8, max_bin 255, 127 leaves: one iteration."""
    from lightgbm_rs_amd.synth import config2_raw_host, sample_mappers
    n, F, nl = 1_000_000, 2000, 127
    X, y = config2_raw_host(n, F=F)
    ms = sample_mappers(X, 255)
    say(f"configs[2] full size {n} x {F}: {sum(m.num_bin for m in ms)} cells")
    trees, scores, init, bins, meta, ub, cfg = _full_chain(X, ms, y, "regression", nl, 0, 0.8)
    del X
    say("device done")
    oscores, otrees = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_REGRESSION, nl, -1, 1,
                                   0.1, quantized=False, feature_fraction=0.8,
                                   feature_fraction_seed=2)
    compare(trees, scores, otrees, oscores, init, "configs[2] full", exact=False)


def test_config4_full_size():
    """2,000,000 x 700 (U(0,1), 30% zeros), Poisson(120) queries,
    lambdarank, quantized int8 gradients, max_bin 255, 255 leaves: three iterations,
    every tree field and every score bit-exact."""
    from lightgbm_rs_amd.synth import config4_raw_host, sample_mappers
    n, F, nl, iters = 2_000_000, 700, 255, 3
    X, rel, groups = config4_raw_host(n, F=F)
    qb = np.concatenate([[0], np.cumsum(groups)]).astype(np.int32)
    ms = sample_mappers(X, 255)
    say(f"configs[4] full size {n} x {F}, {len(groups)} queries, {iters} iterations")
    trees, scores, init, bins, meta, ub, cfg = _full_chain(X, ms, rel, "lambdarank", nl, 4, qb=qb,
                                                           iters=iters)
    del X
    say("device done")
    oscores, otrees = oracle.train(bins, meta, ub, rel, cfg, oracle.OBJECTIVE_LAMBDARANK, nl, -1,
                                   iters, 0.1, quantized=True, query_boundaries=qb)
    compare(trees, scores, otrees, oscores, 0.0, "configs[4] full", exact=True)
