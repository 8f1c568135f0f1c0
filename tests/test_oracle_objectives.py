"""The oracle's L2 regression, LambdaRank and column-sampler restatements pinned on
the reference's fixtures and the real LightGBM 4.6 binary's captures:

  * L2 gradients and BoostFromScore: the hand-computed cases of the reference's own
    unit tests (regression.rs:710-753);
  * Random::Sample: the branch edges (random.rs:179-221); ColSampler: the genuine
    Random::Sample transcription's draw sequence (learner/col_sampler.txt);
  * feature_fraction (per-tree column sampling, feature_fraction_seed 2): every
    tree's set of split features and the raw predictions of the real binary
    (feature_fraction/feature_fraction_golden.json, 5 cells);
  * LambdaRank: the iteration-1 gradients at zero scores bit for bit
    (rank/lambdarank_gh_iter1.txt) and the 10-iteration model of the real binary
    (trees and final raw scores, rank/rank_lambdarank_byq0_es0_model.txt).
A planted mistake in each restated function fails its pin (checked here by
perturbing the inputs the way a wrong term would).
"""
import json
import os

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, feature_mappers, feature_meta
from oracle import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# --- L2 regression -----------------------------------------------------------------
def test_l2_gradients_match_the_reference_unit_case():
    # regression.rs:710-729: grad = f32(score - label), hess = 1
    g, h = oracle.regression_gradients([3.0, -2.5, 0.0, 100.25], [1.0, 0.5, -4.0, 100.0])
    assert g.tolist() == [2.0, -3.0, 4.0, 0.25]
    assert h.tolist() == [1.0] * 4
    # the f64 subtraction before the f32 cast (a f32 subtraction rounds differently)
    s, l = 1.0 + 2.0 ** -30, np.float32(1.0)
    g, _ = oracle.regression_gradients([s], [l])
    assert g[0] == np.float32(s - float(l)) and g[0] != np.float32(np.float32(s) - l)


def test_l2_boost_from_score_is_the_ordered_label_mean():
    assert oracle.regression_boost_from_score([1, 2, 3, 4, 5]) == 3.0  # regression.rs:744-753
    rng = np.random.default_rng(3)
    y = rng.standard_normal(100_001).astype(np.float32) * 1e3
    ref = 0.0
    for v in y.astype(np.float64):  # the sequential f64 fold, then / n
        ref += v
    assert oracle.regression_boost_from_score(y) == ref / len(y)


# --- Random::Sample / ColSampler -----------------------------------------------------
def test_random_sample_branches():
    # random.rs:179-221: K > N or K <= 0 -> empty; K == N -> all; the streaming
    # branch when K > N / log2(K), else the ordered-set branch (sorted, distinct)
    assert len(oracle.random_sample(1, 5, 6)) == 0
    assert len(oracle.random_sample(1, 5, 0)) == 0
    assert oracle.random_sample(1, 5, 5).tolist() == [0, 1, 2, 3, 4]
    for n, k in ((100, 3), (100, 60), (1000, 10), (37, 36)):
        v = oracle.random_sample(11, n, k)
        assert np.all(np.diff(v) > 0) and v.min() >= 0 and v.max() < n
        streaming = k > 1 and k > n / np.log2(k)
        if not streaming:
            assert len(v) == k  # the set branch always yields K values


def test_col_sampler_draw_sequence_golden():
    with open(os.path.join(GOLD, "col_sampler.json")) as f:
        d = json.load(f)
    nf = d["num_features"]
    bt, nodes = oracle.col_sampler_trace(d["feature_fraction"], d["feature_fraction_bynode"],
                                         d["seed"], nf, len(d["nodes"]))
    assert np.flatnonzero(bt).tolist() == d["bytree"]
    for k, want in enumerate(d["nodes"]):
        assert np.flatnonzero(nodes[k]).tolist() == want, k
    # a sampler re-seeded per draw (the reference's fixed defect) repeats the first
    _, first = oracle.col_sampler_trace(d["feature_fraction"], d["feature_fraction_bynode"],
                                        d["seed"], nf, 1)
    assert any(np.flatnonzero(first[0]).tolist() != w for w in d["nodes"][1:])


def _feature_fraction_inputs():
    z = np.load(os.path.join(GOLD, "feature_fraction.npz"))
    X, y = z["X"], z["y"].astype(np.float32)
    ms = feature_mappers(X, max_bin=63, min_data_in_leaf=5)
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    cells, off = [], 0
    for i, ff in enumerate(z["fractions"]):
        trees = []
        for c in z["split_counts"][i]:
            trees.append(sorted(z["split_flat"][off:off + c].tolist()))
            off += c
        cells.append(dict(ff=float(ff), pred=z["pred_bits"][i].view(np.float64), trees=trees))
    return z, bins, meta, ub, y, cells


FF_CELLS = [0, 1, 2, 3, 4]


@pytest.mark.parametrize("cell", FF_CELLS)
def test_feature_fraction_matches_real_binary(cell):
    """Binary boosting, f32 gradients, per-tree column sampling (feature_fraction
    of the cell, seed 2): each tree's split features and the raw predictions."""
    z, bins, meta, ub, y, cells = _feature_fraction_inputs()
    c = cells[cell]
    cfg = GainConfig.make(min_data_in_leaf=5)
    iters = int(z["num_iterations"])
    scores, trees = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_BINARY, 8, -1, iters,
                                 0.1, quantized=False, feature_fraction=c["ff"],
                                 feature_fraction_seed=2)
    assert len(trees) == iters
    for t, want in zip(trees, c["trees"]):
        got = sorted(set(int(v) for v in t["split_feature"][:t["num_leaves"] - 1]))
        assert got == want
    assert np.array_equal(scores.view(np.uint64), c["pred"].view(np.uint64))


def test_feature_fraction_cells_have_teeth():
    """The sampled cells' trees use different feature sets from the unsampled one,
    so the cell tests cannot pass on a learner that ignored feature_fraction; and
    drawing the Init sample for tree 0 (one draw off) changes the sets."""
    z, bins, meta, ub, y, cells = _feature_fraction_inputs()
    full = [c for c in cells if c["ff"] == 1.0][0]
    for c in cells:
        if c["ff"] < 1.0:
            assert c["trees"] != full["trees"], c["ff"]
    c = [c for c in cells if c["ff"] == 0.5][0]
    cfg = GainConfig.make(min_data_in_leaf=5)
    # a different seed stands in for a shifted draw sequence
    _, trees = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_BINARY, 8, -1, 8, 0.1,
                            quantized=False, feature_fraction=0.5, feature_fraction_seed=3)
    got = [sorted(set(int(v) for v in t["split_feature"][:t["num_leaves"] - 1])) for t in trees]
    assert got != c["trees"]


# --- LambdaRank ----------------------------------------------------------------------
def _rank():
    with open(os.path.join(GOLD, "lambdarank.json")) as f:
        return json.load(f)


def test_lambdarank_iteration1_gradients_bit_exact():
    d = _rank()
    y = np.array(d["label_bits"], dtype=np.uint32).view(np.float32)
    qb = np.array(d["query_boundaries"], dtype=np.int32)
    g, h = oracle.lambdarank_gradients(np.zeros(len(y)), y, qb, d["sigmoid"], d["lambdarank_norm"],
                                       d["truncation_level"])
    assert g.view(np.uint32).tolist() == d["gh_iter1"]["GRAD"]
    assert h.view(np.uint32).tolist() == d["gh_iter1"]["HESS"]
    # the truncation level and the normalisation both bite on this corpus
    g2, _ = oracle.lambdarank_gradients(np.zeros(len(y)), y, qb, 1.0, True, 4)
    g3, _ = oracle.lambdarank_gradients(np.zeros(len(y)), y, qb, 1.0, False, 5)
    assert not np.array_equal(g2, g) and not np.array_equal(g3, g)


def test_lambdarank_gradients_at_distinct_scores():
    """The real binary's final raw scores (no ties): every row's lambda is a sum over
    its pairs; check the pair structure against a brute-force pass written from the
    pairwise definition (sorted ranks, gains 2^l - 1, discounts 1/log2(2 + r))."""
    d = _rank()
    y = np.array(d["label_bits"], dtype=np.uint32).view(np.float32)
    qb = np.array(d["query_boundaries"], dtype=np.int32)
    s = np.array(d["score_bits"], dtype=np.uint64).view(np.float64)
    g, h = oracle.lambdarank_gradients(s, y, qb, 1.0, False, 30)
    for q in range(len(qb) - 1):
        a, b = qb[q], qb[q + 1]
        ss, ll = s[a:b], y[a:b]
        order = np.argsort(-ss, kind="stable")
        rank = np.empty(len(ss), int)
        rank[order] = np.arange(len(ss))
        labels_sorted = np.sort(ll)[::-1][:30]
        maxdcg = sum((2.0 ** l - 1) / np.log2(2 + i) for i, l in enumerate(labels_sorted))
        lam = np.zeros(len(ss))
        for i in range(len(ss)):
            for j in range(len(ss)):
                if ll[i] <= ll[j]:
                    continue
                dpn = (2.0 ** ll[i] - 2.0 ** ll[j]) * abs(1 / np.log2(2 + rank[i]) -
                                                        1 / np.log2(2 + rank[j])) / maxdcg
                p = 1.0 / (1.0 + np.exp(ss[i] - ss[j]))
                lam[i] -= p * dpn
                lam[j] += p * dpn
        # the 2^20-bin sigmoid table quantises the score gap to 50 / 2^20
        np.testing.assert_allclose(g[a:b], lam, rtol=1e-4, atol=1e-5)


def test_lambdarank_nan_label_follows_rust_casts():
    """A NaN relevance label passes check_labels (dcg_calculator.rs:112-137: NaN - 0 is
    NaN, and `NaN > eps`, `NaN < 0` are false), indexes the label gains as 0 (Rust's
    saturating `as usize`), and in the pair loop (rank.rs:317-336) compares neither
    equal to nor greater than the other label, so the later-ranked document of the
    pair is taken as the high one.  Two documents, scores (1, 0), labels (2, NaN):
    high = doc 1 (gain 0), low = doc 0 (gain 3), so dcg_gap = -3 and the pair's
    hessian term is negative (a NaN read as label 0 would give a positive one)."""
    s = np.array([1.0, 0.0])
    y = np.array([2.0, np.nan], np.float32)
    qb = np.array([0, 2], np.int32)
    g, h = oracle.lambdarank_gradients(s, y, qb, 1.0, True, 30)
    # max DCG of labels (2, 0) at k = 2: gain 3 at discount 1; pair at ranks (1, 0)
    paired = abs(1.0 / np.log2(3.0) - 1.0)
    dpn = (-3.0 * paired * (1.0 / 3.0)) / (float(np.float32(0.01)) + 1.0)
    # the sigmoid table entry of delta = s[1] - s[0] = -1 (2^20 bins over [-25, 25])
    f = 2.0 ** 20 / 50.0
    sc = int((-1.0 + 25.0) * f) / f - 25.0
    p = 1.0 / (1.0 + np.exp(sc))
    pl = p * -(1.0 * dpn)
    ph = p * (1.0 - p) * dpn
    assert g[0] == np.float32(-np.float32(pl)) and g[1] == np.float32(pl), (g, pl)
    assert h[0] == np.float32(ph) and h[1] == np.float32(ph) and h[0] < 0, (h, ph)
    # NaN labels in a larger query: every label's f32 comparisons stay the reference's
    rng = np.random.default_rng(1)
    y2 = rng.integers(0, 5, 50).astype(np.float32)
    y2[[3, 17, 18]] = np.nan
    g2, h2 = oracle.lambdarank_gradients(rng.normal(size=50), y2, np.array([0, 50], np.int32))
    assert np.all(np.isfinite(g2)) and np.all(np.isfinite(h2))


def test_lambdarank_model_matches_real_binary():
    d = _rank()
    X = np.array(d["X"], dtype=np.float64)
    y = np.array(d["label_bits"], dtype=np.uint32).view(np.float32)
    qb = np.array(d["query_boundaries"], dtype=np.int32)
    ms = feature_mappers(X, max_bin=255, min_data_in_bin=1, min_data_in_leaf=1)
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    cfg = GainConfig.make(min_data_in_leaf=1, min_sum_hessian_in_leaf=1e-3)
    scores, trees = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_LAMBDARANK,
                                 d["num_leaves"], -1, d["num_iterations"], d["learning_rate"],
                                 quantized=False, query_boundaries=qb, sigmoid=d["sigmoid"],
                                 lambdarank_norm=d["lambdarank_norm"],
                                 truncation_level=d["truncation_level"])
    assert len(trees) == len(d["trees"])
    for i, (t, gt) in enumerate(zip(trees, d["trees"])):
        nl = int(gt["num_leaves"][0])
        assert t["num_leaves"] == nl, i
        assert t["split_feature"][:nl - 1].tolist() == [int(v) for v in gt["split_feature"]], i
        assert t["leaf_count"][:nl].tolist() == [int(v) for v in gt["leaf_count"]], i
        lv = np.array([float(v) for v in gt["leaf_value"]])
        assert np.array_equal(t["leaf_value"][:nl].view(np.uint64), lv.view(np.uint64)), i
        # the binary writes kZeroThreshold as the f32 1e-35f widened; the reference's
        # binning (and this library's) keeps the f64 1e-35 (types.rs:35)
        thr = np.array([1e-35 if float(v) == float(np.float32(1e-35)) else float(v)
                        for v in gt["threshold"]])
        assert np.array_equal(t["threshold"][:nl - 1], thr), i
    want = np.array(d["score_bits"], dtype=np.uint64).view(np.float64)
    assert np.array_equal(scores.view(np.uint64), want.view(np.uint64))
