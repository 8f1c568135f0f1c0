"""Edge inputs of the device objectives and tree outputs, against the oracle.

  * LambdaRank with NaN relevance labels: the reference lets them through
    DCGCalculator::check_labels (every comparison with NaN is false) and indexes the
    label gains with Rust's saturating `as usize` (NaN -> 0) while the pair loop still
    compares the f32 labels (lgbm-metric/src/dcg_calculator.rs:112-137,
    lgbm-objective/src/rank.rs:317-336): gradients bit-exact with the oracle;
  * LambdaRank queries of 1639 and 2048 rows (the kernel's LDS above 64 KiB);
  * a tree output whose categorical bitset capacity is too small is refused before any
    work: the resident scores stay as they were and the next call trains normally.
"""
import ctypes as C

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend, feature_meta, feature_mappers
from lightgbm_rs_amd._abi import TreeBuffers
from lightgbm_rs_amd.synth import config4_binned
from oracle import oracle

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _rank_grads_at_trained_scores(bins, meta, ub, rel, qb, iters=2, qbins=4):
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.set_labels(rel, 0.0)
        b.set_lambdarank(qb)
        cfg = GainConfig.make(min_data_in_leaf=20)
        for i in range(iters):
            b.train_iter(i, cfg, 31, -1, 0.1, qbins, True)
        s = b.scores()
        b.train_iter(iters, cfg, 31, -1, 0.1, qbins, True)  # evaluates the gradients at s
        g, h = b.gradients()
    finally:
        b.close()
    return s, g, h


def test_lambdarank_nan_labels_match_oracle():
    n, F = 20_000, 24
    bins, meta, ub, rel, groups = config4_binned(n, F=F, seed=0x5EED0045)
    qb = np.concatenate([[0], np.cumsum(groups)]).astype(np.int32)
    rel = rel.astype(np.float32).copy()
    rng = np.random.default_rng(7)
    nan_rows = rng.choice(n, n // 50, replace=False)
    rel[nan_rows] = np.nan
    # one query holding only NaN labels, one with a single non-NaN label
    rel[qb[3]:qb[4]] = np.nan
    rel[qb[5]:qb[6]] = np.nan
    rel[qb[5]] = 3.0
    say(f"lambdarank NaN labels n={n} nan={int(np.isnan(rel).sum())}")
    # a NaN-labelled pair can carry a negative hessian term (the quantized learner
    # refuses those): the trees grow from f32 gradients
    s, g, h = _rank_grads_at_trained_scores(bins, meta, ub, rel, qb, qbins=0)
    og, oh = oracle.lambdarank_gradients(s, rel, qb)
    assert np.array_equal(g.view(np.uint32), og.view(np.uint32))
    assert np.array_equal(h.view(np.uint32), oh.view(np.uint32))
    assert np.any(g[nan_rows] != 0.0), "NaN-labelled documents take part in pairs"
    assert np.any(h < 0.0), "the reference's NaN pairs give negative hessian terms"


@pytest.mark.parametrize("qlen", [1639, 2048])
def test_lambdarank_long_queries_match_oracle(qlen):
    F = 16
    groups = np.array([qlen, 700, qlen, 37, qlen - 1], dtype=np.int64)
    n = int(groups.sum())
    bins, meta, ub, rel, _ = config4_binned(n, F=F, seed=0x5EED0046 + qlen)
    qb = np.concatenate([[0], np.cumsum(groups)]).astype(np.int32)
    say(f"lambdarank queries of {qlen} rows, n={n}")
    s, g, h = _rank_grads_at_trained_scores(bins, meta, ub, rel, qb)
    og, oh = oracle.lambdarank_gradients(s, rel, qb)
    assert np.array_equal(g.view(np.uint32), og.view(np.uint32))
    assert np.array_equal(h.view(np.uint32), oh.view(np.uint32))


def test_categorical_capacity_refused_before_work():
    n, nl = 40_000, 31
    rng = np.random.default_rng(3)
    Xn = rng.standard_normal((4, n))
    codes = rng.integers(0, 12, (2, n))
    Xc = (codes * 20011 + 7).astype(np.float64)  # category values up to 220128
    eff = rng.standard_normal((2, 12))
    logit = Xn[0] + eff[0][codes[0]] + eff[1][codes[1]]
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-logit))).astype(np.float32)
    X = np.concatenate([Xn, Xc]).T
    ms = feature_mappers(X, categorical_features=[4, 5], max_bin=63, min_data_in_leaf=20)
    be = HipBackend(0)
    try:
        be.upload_raw(X, ms)
        need = be.cat_threshold_words(nl)
        assert need == (nl - 1) * (220128 // 32 + 1), need
        init = oracle.boost_from_score(y)
        be.set_labels(y, init)
        cfg = GainConfig.make(min_data_in_leaf=20)
        cfg.min_data_per_group = 50
        before = be.scores().copy()
        small = TreeBuffers(nl, 64 * (nl - 1))
        rc = be.lib.lgbm_hip_train_iter_binary(be.ctx, C.c_int32(0), C.byref(cfg), C.c_int32(nl),
                                               C.c_int32(-1), C.c_double(0.1), C.c_int32(4),
                                               C.c_int32(1), C.byref(small.out))
        assert rc == -1, rc  # LENGTH_MISMATCH
        assert "cat_threshold" in be._err(be.ctx)
        assert np.array_equal(be.scores(), before), "a refused call changed the scores"
        t = be.train_iter_binary(0, cfg, nl, -1, 0.1)
        assert int(t["num_cat"]) > 0, "the corpus grows categorical splits"
        bins = be.get_bins()
        meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f,
                             bin_type=m.bin_type) for f, m in enumerate(ms)]
        vals = np.concatenate([m.upper_bounds if m.bin_type == 0 else m.categories.astype(np.float64)
                               for m in ms])
        oscores, otrees = oracle.train_binary(bins, meta, vals, y, cfg, nl, -1, 1, 0.1)
        assert np.array_equal(be.scores().view(np.uint64), oscores.view(np.uint64))
        assert np.array_equal(np.asarray(t["cat_threshold"]), np.asarray(otrees[0]["cat_threshold"]))
    finally:
        be.close()
