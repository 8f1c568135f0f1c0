"""Softmax multiclass boosting and categorical splits on the device (configs[3]'s
path) against the oracle and the reference's real-binary multiclass goldens.

  * the multiclass spine (boosting_parity.rs:1259-1300): five iterations through
    lgbm_hip_train_iter_multiclass; every iteration's class-major raw scores and every
    tree's leaf values bit-exact with the real binary;
  * softmax gradients on the device vs MulticlassSoftmax::get_gradients (oracle) on
    the scores the device reached;
  * categorical splits with quantized gradients (exact integer histograms): binary
    boosting with categorical features, trees (category bitsets included), layouts and
    scores bit-exact with the oracle;
  * configs[3]'s workload (10 classes, 80 numerical + 20 categorical features of 32
    levels, max_bin 255, 127 leaves, f32 gradients) at 200k rows and at its full 2M
    rows: every tree's structure (features, thresholds, category bitsets, children,
    counts) identical to the oracle's, leaf values and scores within 1e-9 relative
    (the stated f32-gradient bar is 1e-5 relative).
"""
import json
import os

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend, feature_mappers, feature_meta
from lightgbm_rs_amd.synth import config3_binned
from oracle import oracle

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
K_EPS = float(np.float32(1e-15))


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


def bits(a):
    return np.ascontiguousarray(a, np.float64).view(np.uint64)


def _mrz(v):
    z = float(np.float32(1e-35))
    return np.where((v >= -z) & (v <= z), 0.0, v)


def _constant_tree(v):
    return {"num_leaves": 1, "leaf_value": np.array([v], np.float64)}


def device_multiclass(be, y, K, cfg, num_leaves, iters, lr, quant_bins=0):
    """The GBDT loop (gbdt.rs:691-1373) around lgbm_hip_train_iter_multiclass: the
    BoostFromAverage init per class, class_need_train, constant trees for classes that
    do not split, add_bias on the first iteration, and the stop when no class splits.
    Returns (trees, per-iteration class-major scores)."""
    n = len(y)
    prior = np.bincount(y.astype(np.int64), minlength=K) / n
    init = np.log(np.maximum(prior, K_EPS))
    applied = np.where(np.abs(init) > K_EPS, init, 0.0)
    need = [0 if (p <= K_EPS or p >= 1.0 - K_EPS) else 1 for p in np.abs(prior)]
    be.set_labels_multiclass(y, K, applied)
    trees, score_iters = [], []
    for it in range(iters):
        ts = be.train_iter_multiclass(it, cfg, num_leaves, -1, lr, quant_bins, True, need)
        if not any(t["num_leaves"] > 1 for t in ts):
            if it == 0:
                trees.extend(_constant_tree(init[k]) for k in range(K))
                score_iters.append(be.scores())
            break
        for k, t in enumerate(ts):
            if t["num_leaves"] <= 1:
                t = _constant_tree(init[k] if it == 0 else 0.0)
            elif it == 0 and abs(init[k]) > K_EPS:
                t["leaf_value"] = _mrz(t["leaf_value"] + init[k])
                t["internal_value"] = _mrz(t["internal_value"] + init[k])
            trees.append(t)
        score_iters.append(be.scores())
    return trees, score_iters


STRUCT = ("split_feature", "threshold_in_bin", "decision_type", "left_child", "right_child",
          "leaf_count", "internal_count", "num_cat", "cat_boundaries", "cat_threshold")


def compare_tree(t, o, tag, exact=True, rtol=1e-9):
    assert t["num_leaves"] == o["num_leaves"], tag
    if o["num_leaves"] <= 1:
        assert np.allclose(t["leaf_value"][:1], o["leaf_value"][:1], rtol=rtol, atol=0), tag
        return
    for k in STRUCT:
        assert np.array_equal(np.asarray(t[k]), np.asarray(o[k])), (tag, k)
    for k in ("threshold", "leaf_value", "internal_value", "internal_weight", "leaf_weight"):
        a, b = np.asarray(t[k], np.float64), np.asarray(o[k], np.float64)
        if exact:
            assert np.array_equal(bits(a), bits(b)), (tag, k)
        else:
            assert np.allclose(a, b, rtol=rtol, atol=1e-300), (tag, k, np.max(np.abs(a - b)))


# --- the reference's real-binary multiclass spine --------------------------------
def test_multiclass_spine_on_device(be):
    with open(os.path.join(GOLD, "multiclass_spine.json")) as f:
        d = json.load(f)
    say("multiclass spine on device")
    X = np.array(d["X"], dtype=np.float64)
    y = np.array(d["labels"], dtype=np.float32)
    ms = feature_mappers(X, max_bin=255, min_data_in_bin=1, min_data_in_leaf=1)
    be.upload_raw(X, ms)
    cfg = GainConfig.make(min_data_in_leaf=1)
    trees, score_iters = device_multiclass(be, y, d["num_class"], cfg, d["num_leaves"],
                                           d["num_iterations"], d["learning_rate"])
    for i, s in enumerate(score_iters):
        assert bits(s).tolist() == d["score_bits"][i], f"iteration {i + 1}"
    assert len(trees) == len(d["trees"])
    for i, (t, g) in enumerate(zip(trees, d["trees"])):
        assert t["num_leaves"] == int(g["num_leaves"][0]), i
        lv = t["leaf_value"][:t["num_leaves"]]
        assert bits(lv).tolist() == bits([float(x) for x in g["leaf_value"]]).tolist(), i


def test_softmax_gradients_match_oracle(be):
    n, K = 60_000, 10
    say(f"softmax gradients n={n} K={K}")
    bins, meta, vals, y, cat, X, ms = config3_binned(n, seed=11)
    be.upload_resident_bins(bins, meta, vals)
    cfg = GainConfig.make(min_data_in_leaf=20)
    device_multiclass(be, y, K, cfg, 31, 3, 0.3)
    s = be.scores()  # the scores three iterations reached
    be.train_iter_multiclass(3, cfg, 2, -1, 0.1, 0, True)  # evaluates the gradients at s
    g, h = be.multiclass_gradients()
    og, oh = oracle.multiclass_gradients(s, y, K)
    assert g.shape == (K * n,) and h.shape == (K * n,)
    assert np.array_equal(g.view(np.uint32), og.view(np.uint32))
    assert np.array_equal(h.view(np.uint32), oh.view(np.uint32))


# --- categorical splits, exact (quantized) ------------------------------------------
def _cat_binary_data(n, seed):
    rng = np.random.default_rng(seed)
    n_num, n_cat, levels = 12, 8, 12
    Xn = rng.standard_normal((n_num, n)).astype(np.float32)
    Xc = rng.integers(0, levels, (n_cat, n)).astype(np.float32)
    eff = rng.standard_normal((n_cat, levels)).astype(np.float32)
    logit = Xn[0] - 0.5 * Xn[1] + sum(eff[j][Xc[j].astype(np.int64)] for j in range(n_cat))
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-logit))).astype(np.float32)
    X = np.concatenate([Xn, Xc]).T.astype(np.float64)
    return X, y, list(range(n_num, n_num + n_cat))


def test_categorical_quantized_binary_matches_oracle(be):
    n, iters, nl = 100_000, 4, 63
    say(f"categorical quantized binary n={n}")
    X, y, cat = _cat_binary_data(n, 5)
    ms = feature_mappers(X, categorical_features=cat, max_bin=63, min_data_in_leaf=20)
    be.upload_raw(X, ms)
    bins = be.get_bins()
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f,
                         bin_type=m.bin_type) for f, m in enumerate(ms)]
    vals = np.concatenate([m.upper_bounds if m.bin_type == 0 else m.categories.astype(np.float64)
                           for m in ms])
    init = oracle.boost_from_score(y)
    be.set_labels(y, init)
    cfg = GainConfig.make(min_data_in_leaf=20)
    cfg.min_data_per_group = 50
    trees = [be.train_iter_binary(i, cfg, nl, -1, 0.1) for i in range(iters)]
    scores = be.scores()
    oscores, otrees = oracle.train_binary(bins, meta, vals, y, cfg, nl, -1, iters, 0.1)
    assert sum(int(t["num_cat"]) for t in otrees) > 0, "the corpus grows categorical splits"
    assert len(trees) == len(otrees)
    for i, (t, o) in enumerate(zip(trees, otrees)):
        t = dict(t)
        if i == 0:
            t["leaf_value"] = _mrz(t["leaf_value"] + init)
            t["internal_value"] = _mrz(t["internal_value"] + init)
        compare_tree(t, o, ("cat binary", i), exact=True)
        assert np.array_equal(np.asarray(t["split_gain"]), np.asarray(o["split_gain"])), i
    assert np.array_equal(bits(scores), bits(oscores))


# --- configs[3] ---------------------------------------------------------------------
def _config3_case(be, n, iters, seed):
    K, nl = 10, 127
    bins, meta, vals, y, cat, X, ms = config3_binned(n, seed=seed)
    say(f"configs[3] n={n} iterations={iters}: binned, {sum(m.num_bin for m in meta)} cells")
    be.upload_resident_bins(bins, meta, vals)
    cfg = GainConfig.make(min_data_in_leaf=20)
    trees, score_iters = device_multiclass(be, y, K, cfg, nl, iters, 0.1)
    say("device done")
    oscores, otrees = oracle.train_multiclass(bins, meta, vals, y, K, cfg, nl, -1, iters, 0.1)
    say("oracle done")
    assert sum(int(t["num_cat"]) for t in otrees) > 0
    assert len(trees) == len(otrees)
    for i, (t, o) in enumerate(zip(trees, otrees)):
        compare_tree(t, o, ("configs[3]", n, i), exact=False)
    s = score_iters[-1]
    lv_exact = all(np.array_equal(bits(t["leaf_value"]), bits(o["leaf_value"]))
                   for t, o in zip(trees, otrees))
    say(f"leaf values bit-exact: {lv_exact}; scores bit-exact: "
        f"{np.array_equal(bits(s), bits(oscores))}, max |diff| {np.max(np.abs(s - oscores)):.3g}")
    assert np.allclose(s, oscores, rtol=1e-9, atol=1e-12), np.max(np.abs(s - oscores))


def test_config3_workload_matches_oracle(be):
    _config3_case(be, 200_000, 2, 0x5EED0003)


def test_config3_full_size_matches_oracle(be):
    _config3_case(be, 2_000_000, 2, 0x5EED0003)
