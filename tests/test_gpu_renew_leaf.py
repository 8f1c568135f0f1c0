"""quant_train_renew_leaf on the device (lgbm_hip_set_quant_renew_leaf) against the
oracle's boosting loops: after each quantized tree, every leaf output recomputed from the
original gradients by an ordered f64 fold over the leaf's rows in partition order
(gbdt.rs:1194-1212, learner.rs:4411-4429).  The fold's order is kept on the device (one
thread per leaf over the exported layout), so trees and scores are bit-exact: binary
(with and without the lookahead), lambdarank, and softmax multiclass with its
per-class trees.
"""
import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend
from lightgbm_rs_amd.synth import config1_like, config3_binned, config4_binned
from oracle import oracle

pytestmark = pytest.mark.gpu
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


@pytest.mark.parametrize("lookahead", [False, True])
def test_renew_binary_matches_oracle(lookahead):
    n, nl, iters = 200_000, 63, 3
    bins, meta, ub, y = config1_like(n, seed=31)
    cfg = GainConfig.make(min_data_in_leaf=20, lambda_l1=0.05, lambda_l2=0.5)
    init = oracle.boost_from_score(y)
    say(f"renew binary n={n} lookahead={lookahead}")
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, ub)
        be.set_labels(y, init)
        be.set_quant_renew_leaf(True)
        be.set_lookahead(lookahead)
        trees = [be.train_iter_binary(i, cfg, nl, -1, 0.1, 4, True) for i in range(iters)]
        scores = be.scores()
    finally:
        be.close()
    oscores, otrees = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_BINARY, nl, -1, iters,
                                   0.1, quantized=True, quant_bins=4, stochastic=True,
                                   quant_renew_leaf=True)
    _, plain = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_BINARY, nl, -1, 1, 0.1,
                            quantized=True, quant_bins=4, stochastic=True)
    assert not np.array_equal(bits(plain[0]["leaf_value"]), bits(otrees[0]["leaf_value"]))
    for i, (t, o) in enumerate(zip(trees, otrees)):
        t = dict(t)
        if i == 0:
            t["leaf_value"] = _mrz(t["leaf_value"] + init)
            t["internal_value"] = _mrz(t["internal_value"] + init)
        _same_tree(t, o, ("binary", i))
    assert np.array_equal(bits(scores), bits(oscores))


def test_renew_lambdarank_matches_oracle():
    n, F, nl, iters = 40_000, 24, 63, 2
    bins, meta, ub, rel, groups = config4_binned(n, F=F, seed=0x5EED0047)
    qb = np.concatenate([[0], np.cumsum(groups)]).astype(np.int32)
    cfg = GainConfig.make(min_data_in_leaf=20)
    say(f"renew lambdarank n={n}")
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, ub)
        be.set_labels(rel, 0.0)
        be.set_lambdarank(qb)
        be.set_quant_renew_leaf(True)
        trees = [be.train_iter(i, cfg, nl, -1, 0.1, 4, True) for i in range(iters)]
        scores = be.scores()
    finally:
        be.close()
    oscores, otrees = oracle.train(bins, meta, ub, rel, cfg, oracle.OBJECTIVE_LAMBDARANK, nl, -1,
                                   iters, 0.1, quantized=True, query_boundaries=qb,
                                   quant_renew_leaf=True)
    for i, (t, o) in enumerate(zip(trees, otrees)):
        _same_tree(t, o, ("lambdarank", i))
    assert np.array_equal(bits(scores), bits(oscores))


def test_renew_multiclass_matches_oracle():
    n, K, nl, iters = 60_000, 10, 31, 2
    bins, meta, vals, y, cat, _, _ = config3_binned(n, seed=0x5EED0048)
    cfg = GainConfig.make(min_data_in_leaf=20)
    say(f"renew multiclass n={n} K={K}")
    prior = np.bincount(y.astype(np.int64), minlength=K) / n
    init = np.log(np.maximum(prior, K_EPS))
    applied = np.where(np.abs(init) > K_EPS, init, 0.0)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, vals)
        be.set_labels_multiclass(y, K, applied)
        be.set_quant_renew_leaf(True)
        trees = []
        for it in range(iters):
            ts = be.train_iter_multiclass(it, cfg, nl, -1, 0.1, 4, True, [1] * K)
            for k, t in enumerate(ts):
                t = dict(t)
                if it == 0 and abs(init[k]) > K_EPS:
                    t["leaf_value"] = _mrz(t["leaf_value"] + init[k])
                    t["internal_value"] = _mrz(t["internal_value"] + init[k])
                trees.append(t)
        scores = be.scores()
    finally:
        be.close()
    oscores, otrees = oracle.train_multiclass(bins, meta, vals, y, K, cfg, nl, -1, iters, 0.1,
                                              quantized=True, quant_bins=4, stochastic=True,
                                              quant_renew_leaf=True)
    assert len(trees) == len(otrees) == K * iters
    for i, (t, o) in enumerate(zip(trees, otrees)):
        _same_tree(t, o, ("multiclass", i))
    assert np.array_equal(bits(scores), bits(oscores))
