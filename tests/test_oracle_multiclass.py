"""Pin the oracle's softmax objective and multiclass boosting loop on the reference's
real-binary multiclass goldens (boosting_parity.rs:110-170, 1259-1300; CPU only).

The corpus is binned with the library's own BinMapper (the same FindBin the binary
ran), then trained for 1..5 iterations: every iteration's class-major raw scores,
the 15 trees and the iteration-1 / iteration-4 gradients match the real binary's
bits.
"""
import json
import os

import numpy as np
import pytest

from lightgbm_rs_amd._abi import GainConfig
from oracle import oracle

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def spine():
    with open(os.path.join(GOLD, "multiclass_spine.json")) as f:
        return json.load(f)


def _inputs(d):
    from lightgbm_rs_amd import feature_mappers, feature_meta
    X = np.array(d["X"], dtype=np.float64)
    # boosting_oracle_capture.py:110-125: max_bin 255, min_data_in_bin 1
    ms = feature_mappers(X, max_bin=255, min_data_in_bin=1, min_data_in_leaf=d["min_data_in_leaf"])
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    cfg = GainConfig.make(min_data_in_leaf=d["min_data_in_leaf"])
    return bins, meta, ub, cfg, np.array(d["labels"], dtype=np.float32)


def _train(d, iters):
    bins, meta, ub, cfg, y = _inputs(d)
    return oracle.train_multiclass(bins, meta, ub, y, d["num_class"], cfg, d["num_leaves"], -1,
                                   iters, d["learning_rate"])


def _bits(a):
    return np.asarray(a, dtype=np.float64).view(np.uint64).tolist()


@pytest.mark.parametrize("iters", [1, 2, 3, 4, 5])
def test_scores_bit_exact_per_iteration(spine, iters):
    scores, trees = _train(spine, iters)
    assert len(trees) == iters * spine["num_class"]
    assert _bits(scores) == spine["score_bits"][iters - 1]


def test_trees_match_model_text(spine):
    _, trees = _train(spine, spine["num_iterations"])
    gold = spine["trees"]
    assert len(trees) == len(gold) == 15
    for i, (t, g) in enumerate(zip(trees, gold)):
        assert t["num_leaves"] == int(g["num_leaves"][0]), i
        assert t["split_feature"].tolist() == [int(x) for x in g["split_feature"]], i
        assert t["decision_type"].tolist() == [int(x) for x in g["decision_type"]], i
        assert t["left_child"].tolist() == [int(x) for x in g["left_child"]], i
        assert t["right_child"].tolist() == [int(x) for x in g["right_child"]], i
        assert t["leaf_count"].tolist() == [int(x) for x in g["leaf_count"]], i
        # the zero bin's bound: the reference's K_ZERO_THRESHOLD is the f64 1e-35
        # (lgbm-core/src/types.rs:35) where the C++ binary writes the widened f32 1e-35f
        gt = [1e-35 if float(x) == float(np.float32(1e-35)) else float(x) for x in g["threshold"]]
        assert _bits(t["threshold"]) == _bits(gt), i
        # leaf values: shrunk, with the first iteration's init folded in (add_bias)
        assert _bits(t["leaf_value"]) == _bits([float(x) for x in g["leaf_value"]]), i


def test_gradients_iteration_1_and_4(spine):
    _, _, _, _, y = _inputs(spine)
    K, n = spine["num_class"], len(y)
    init = np.log(np.maximum(np.bincount(y.astype(int), minlength=K) / n, 1e-15))
    s0 = np.repeat(init, n)
    g, h = oracle.multiclass_gradients(s0, y, K)
    assert g.view(np.uint32).tolist() == spine["gh_iter1"]["GRAD"]
    assert h.view(np.uint32).tolist() == spine["gh_iter1"]["HESS"]
    s3, _ = _train(spine, 3)  # the scores iteration 4 starts from
    g, h = oracle.multiclass_gradients(s3, y, K)
    assert g.view(np.uint32).tolist() == spine["gh_iter4"]["GRAD"]
    assert h.view(np.uint32).tolist() == spine["gh_iter4"]["HESS"]


def test_multiclass_goldens_have_teeth(spine):
    """The goldens tell apart the plausible slips: hessians without the K/(K-1)
    factor, a row-major score layout, and gradients without the label term."""
    _, _, _, _, y = _inputs(spine)
    K, n = spine["num_class"], len(y)
    s3, _ = _train(spine, 3)
    g, h = oracle.multiclass_gradients(s3, y, K)
    gold_h = np.array(spine["gh_iter4"]["HESS"], dtype=np.uint32).view(np.float32)
    gold_g = np.array(spine["gh_iter4"]["GRAD"], dtype=np.uint32).view(np.float32)
    p = g.astype(np.float64) + (np.repeat(np.arange(K), n) == np.tile(y.astype(int), K))
    assert not np.array_equal((p * (1 - p)).astype(np.float32), gold_h)
    g_rm, _ = oracle.multiclass_gradients(s3.reshape(K, n).T.reshape(-1), y, K)
    assert not np.array_equal(g_rm, gold_g)
    assert not np.array_equal(p.astype(np.float32), gold_g)
