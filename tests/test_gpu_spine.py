"""End to end against the real LightGBM 4.6 binary: the reference's binary spine
(crates/oracle-harness/tests/boosting_parity.rs:56-85, 787-810) — 12 rows x 2
identity-binned features, binary objective with boost_from_average, 10 iterations,
learning_rate 0.1, num_leaves 4, min_data_in_leaf 1, f32 gradients — through this
library's whole path: raw values -> BinMapper (host) -> device bins -> resident
boosting (objective, learner, score update) -> model text -> device prediction.

Pins (all from the real binary's captures): the iteration-1 and iteration-5
gradients (f32 bits) and every iteration's training scores (f64 bits) bit-exact;
every tree block of the model text byte-exact except one known substitution: the
zero bin's bound, which the reference's BinMapper (and this library) writes as the
f64 1e-35 (its binning goldens pin that value) and the real binary as the f32
kZeroThreshold 1.0000000180025095e-35; the transformed predictions within 1e-15."""
import os

import numpy as np
import pytest

from lightgbm_rs_amd import (GainConfig, HipBackend, Model, binary_boost_from_score,
                             feature_mappers)

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_text")
F0 = [0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5]
F1 = [0, 1, 2, 0, 1, 2, 0, 1, 2, 0, 1, 2]
LABELS = [0, 0, 0, 0, 0, 1, 0, 1, 1, 0, 1, 1]


def _bits_lines(name):
    out = {}
    for line in open(os.path.join(GOLD, "spine", name)):
        if line.startswith("#") or not line.strip():
            continue
        toks = line.split()
        key = toks[0] if not toks[0].isdigit() else len(out)
        vals = [int(t) for t in toks if t.isdigit()]
        out[key] = np.array(vals, dtype=np.uint64)
    return out


def _tree_blocks(text):
    body = text.split("\n\n", 1)[1].split("end of trees")[0]
    return ["Tree=" + b for b in body.split("Tree=")[1:]]


def test_binary_spine_matches_lightgbm():
    print("binary spine end to end", flush=True)
    X = np.array([F0, F1], dtype=np.float64).T
    y = np.array(LABELS, dtype=np.float32)
    init = binary_boost_from_score(y)
    assert init == -0.33647223662121273  # the capture's `init=` (binary_gh_iterN.txt)
    ms = feature_mappers(X, max_bin=255, min_data_in_bin=1, bin_construct_sample_cnt=1000000,
                         data_random_seed=8662)
    be = HipBackend(0)
    try:
        be.upload_raw(X, ms)
        be.set_labels(y, init)
        cfg = GainConfig.make(min_data_in_leaf=1, min_sum_hessian_in_leaf=1e-3)
        m = Model.create(num_class=1, max_feature_idx=1, objective="binary sigmoid:1",
                         feature_infos="[0:5] [0:2]")
        scores = _bits_lines("binary_scores.txt")
        gh1, ghn = _bits_lines("binary_gh_iter1.txt"), _bits_lines("binary_gh_iterN.txt")
        for i in range(10):
            t = be.train_iter_binary(i, cfg, 4, -1, 0.1, 0, False)
            m.add_tree(t, shrinkage=0.1, bias=init if i == 0 else 0.0)
            if i in (0, 4):
                g, h = be.gradients()
                ref = gh1 if i == 0 else ghn
                assert np.array_equal(g.view(np.uint32), ref["GRAD"].astype(np.uint32)), i
                assert np.array_equal(h.view(np.uint32), ref["HESS"].astype(np.uint32)), i
            assert np.array_equal(be.scores().view(np.uint64), scores[i]), i
        text = m.to_text()
        gold = open(os.path.join(GOLD, "binary_spine.txt")).read()
        ours = _tree_blocks(text)
        theirs = [b.replace("1.0000000180025095e-35", "1e-35") for b in _tree_blocks(gold)]
        assert len(ours) == len(theirs) == 10
        for i, (a, b) in enumerate(zip(ours, theirs)):
            assert a == b, (i, a, b)
        assert text.split("\n")[:9] == gold.split("\n")[:9]  # envelope up to feature_infos
        pred = _bits_lines("binary_spine_pred.txt")[0].view(np.float64)
        got = be.predict(Model(text), X.astype(np.float32), "transformed")[:, 0]
        np.testing.assert_allclose(got, pred, rtol=1e-15, atol=0)
    finally:
        be.close()
