"""num_grad_quant_bins other than 2 and 4 on the device, against the oracle.

Those bin counts train on the dequantized values f32(q * scale) through the fixed-point
path with the exact scale u = ulp(f32(1 * scale)): every dequantized value is an integer
multiple of u, so cells, sums and differences are exact integers and every f64 the
learner sees equals the reference's f64 fold of the same values (gradient_discretizer.rs
:145-188, gbdt.rs:43-62,936-960).  Checked bit for bit: the quantizer's values at 3 to
254 bins, trees and scores of binary / lambdarank / multiclass boosting, the coarse seam
after lgbm_hip_quantize, and the reference's 128-bin quantized corpus (with renewal).
"""
import json
import os

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend, feature_mappers, feature_meta
from lightgbm_rs_amd.backend import HipError
from lightgbm_rs_amd.synth import config1_like, config3_binned, config4_binned
from oracle import oracle

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "quantized")
K_EPS = 1e-15


def say(*a):
    print(*a, flush=True)


def bits(a):
    return np.ascontiguousarray(a, np.float64).view(np.uint64)


def _mrz(v):
    z = float(np.float32(1e-35))
    return np.where((v >= -z) & (v <= z), 0.0, v)


def _same_tree(t, o, tag):
    assert t["num_leaves"] == o["num_leaves"], tag
    for k in o:
        if k == "num_leaves":
            continue
        a, b = np.ascontiguousarray(t[k]), np.ascontiguousarray(o[k])
        assert a.shape == b.shape and a.tobytes() == b.tobytes(), (tag, k)


def _gh(n, seed):
    rng = np.random.default_rng(seed)
    s = rng.normal(0, 1.5, n)
    p = 1 / (1 + np.exp(-s))
    y = (rng.random(n) < p).astype(np.float32)
    return (p - y).astype(np.float32), (p * (1 - p)).astype(np.float32)


@pytest.mark.parametrize("bins", [3, 16, 128, 254])
@pytest.mark.parametrize("stochastic", [False, True])
def test_quantizer_any_bins_matches_oracle(bins, stochastic):
    n = 300_000
    g, h = _gh(n, bins)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(np.zeros((1, n), np.uint8), [feature_meta(2, 0, 0, None, 0)],
                                np.array([0.5, 1.5]))
        be.upload_resident_grad_hess(g, h)
        _, dg, dh = be.discretize_dequantize_in_place(bins, stochastic, 0x51702010 + bins,
                                                      want_values=True)
    finally:
        be.close()
    og, oh, _, _ = oracle.quantize(g, h, bins=bins, stochastic=stochastic, seed=0x51702010 + bins)
    assert np.array_equal(dg.view(np.uint32), og.view(np.uint32))
    assert np.array_equal(dh.view(np.uint32), oh.view(np.uint32))


@pytest.mark.parametrize("bins,stochastic", [(128, True), (16, False), (3, True)])
def test_binary_boosting_any_bins_matches_oracle(bins, stochastic):
    n, nl, iters = 200_000, 63, 3
    X_bins, meta, ub, y = config1_like(n, seed=40 + bins)
    cfg = GainConfig.make(min_data_in_leaf=20)
    init = oracle.boost_from_score(y)
    say(f"binary boosting bins={bins} stochastic={stochastic}")
    be = HipBackend(0)
    try:
        be.upload_resident_bins(X_bins, meta, ub)
        be.set_labels(y, init)
        trees = [be.train_iter_binary(i, cfg, nl, -1, 0.1, bins, stochastic) for i in range(iters)]
        scores = be.scores()
    finally:
        be.close()
    oscores, otrees = oracle.train(X_bins, meta, ub, y, cfg, oracle.OBJECTIVE_BINARY, nl, -1, iters,
                                   0.1, quantized=True, quant_bins=bins, stochastic=stochastic)
    for i, (t, o) in enumerate(zip(trees, otrees)):
        t = dict(t)
        if i == 0:
            t["leaf_value"] = _mrz(t["leaf_value"] + init)
            t["internal_value"] = _mrz(t["internal_value"] + init)
        _same_tree(t, o, ("binary", bins, i))
    assert np.array_equal(bits(scores), bits(oscores))


def test_grow_tree_after_quantize_128_bins():
    n, nl = 150_000, 127
    X_bins, meta, ub, _ = config1_like(n, seed=44)
    g, h = _gh(n, 45)
    cfg = GainConfig.make(min_data_in_leaf=20)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(X_bins, meta, ub)
        be.upload_resident_grad_hess(g, h)
        be.discretize_dequantize_in_place(128, True, 0x51702010)
        t, lay = be.grow_tree_on_device_with_cfg(cfg, nl, -1)
        with pytest.raises(HipError, match="CAPABILITY"):
            be.construct_int_histogram()
    finally:
        be.close()
    og, oh, _, _ = oracle.quantize(g, h, bins=128, stochastic=True, seed=0x51702010)
    o, olay = oracle.train_tree(X_bins, meta, ub, og, oh, cfg, nl, -1)
    _same_tree(t, o, "grow_tree 128 bins")
    assert np.array_equal(lay["indices"], olay["indices"])


def test_lambdarank_32_bins_matches_oracle():
    n, F, nl, iters = 40_000, 24, 63, 2
    bins, meta, ub, rel, groups = config4_binned(n, F=F, seed=0x5EED0049)
    qb = np.concatenate([[0], np.cumsum(groups)]).astype(np.int32)
    cfg = GainConfig.make(min_data_in_leaf=20)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, ub)
        be.set_labels(rel, 0.0)
        be.set_lambdarank(qb)
        trees = [be.train_iter(i, cfg, nl, -1, 0.1, 32, True) for i in range(iters)]
        scores = be.scores()
    finally:
        be.close()
    oscores, otrees = oracle.train(bins, meta, ub, rel, cfg, oracle.OBJECTIVE_LAMBDARANK, nl, -1,
                                   iters, 0.1, quantized=True, quant_bins=32, query_boundaries=qb)
    for i, (t, o) in enumerate(zip(trees, otrees)):
        _same_tree(t, o, ("lambdarank 32", i))
    assert np.array_equal(bits(scores), bits(oscores))


def test_multiclass_8_bins_matches_oracle():
    n, K, nl, iters = 60_000, 10, 31, 2
    bins, meta, vals, y, _, _, _ = config3_binned(n, seed=0x5EED004A)
    cfg = GainConfig.make(min_data_in_leaf=20)
    prior = np.bincount(y.astype(np.int64), minlength=K) / n
    init = np.log(np.maximum(prior, K_EPS))
    applied = np.where(np.abs(init) > K_EPS, init, 0.0)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, vals)
        be.set_labels_multiclass(y, K, applied)
        trees = []
        for it in range(iters):
            for k, t in enumerate(be.train_iter_multiclass(it, cfg, nl, -1, 0.1, 8, True, [1] * K)):
                t = dict(t)
                if it == 0 and abs(init[k]) > K_EPS:
                    t["leaf_value"] = _mrz(t["leaf_value"] + init[k])
                    t["internal_value"] = _mrz(t["internal_value"] + init[k])
                trees.append(t)
        scores = be.scores()
    finally:
        be.close()
    oscores, otrees = oracle.train_multiclass(bins, meta, vals, y, K, cfg, nl, -1, iters, 0.1,
                                              quantized=True, quant_bins=8, stochastic=True)
    for i, (t, o) in enumerate(zip(trees, otrees)):
        _same_tree(t, o, ("multiclass 8", i))
    assert np.array_equal(bits(scores), bits(oscores))


@pytest.mark.parametrize("renew", [False, True])
def test_reference_128_bin_corpus_on_device(renew):
    """The reference's quantized corpus (512 x 6, num_grad_quant_bins 128, deterministic,
    7 leaves, 10 iterations): the device's scores equal the oracle's bit for bit, and
    the probabilities stay inside the reference's own gate against real LightGBM."""
    z = np.load(os.path.join(GOLD, "quant_binary.npz"))
    p = json.loads(str(z["params"]))["params"]
    X, y = z["X"], z["y"]
    ms = feature_mappers(X, max_bin=p["max_bin"], min_data_in_leaf=p["min_data_in_leaf"])
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    cfg = GainConfig.make(min_data_in_leaf=p["min_data_in_leaf"])
    init = oracle.boost_from_score(y)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, ub)
        be.set_labels(y, init)
        be.set_quant_renew_leaf(renew)
        for i in range(10):
            be.train_iter_binary(i, cfg, p["num_leaves"], -1, p["learning_rate"], 128, False)
        scores = be.scores()
    finally:
        be.close()
    oscores, _ = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_BINARY, p["num_leaves"], -1,
                              10, p["learning_rate"], quantized=True, quant_bins=128,
                              stochastic=False, quant_renew_leaf=renew)
    assert np.array_equal(bits(scores), bits(oscores))
    prob = 1.0 / (1.0 + np.exp(-scores))
    want = z["pred_renew"] if renew else z["pred"]
    assert np.max(np.abs(prob - want)) < 1e-2
