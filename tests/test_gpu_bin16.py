"""2-byte bin columns (BinColumn::U16, lgbm-compute/src/lib.rs:75-211): features of more
than 256 bins select the wide row layout with 2-byte bins.

  * quantized binary boosting over features of up to ~4000 bins (numerical, NaN
    bins, and 1-byte-sized categorical columns beside them): trees, split gains and
    scores bit-exact with the oracle on the same u16 bins;
  * a tree from f32 gradients with its partition layout against the oracle;
  * device binning of a raw table with 2-byte mappers (lgbm_hip_upload_raw) equal to
    the host mappers' bins;
  * u16 input whose features all fit a byte trains exactly as the u8 upload.
"""
import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend, feature_mappers, feature_meta
from oracle import oracle

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def bits(a):
    return np.ascontiguousarray(a, np.float64).view(np.uint64)


def _mrz(v):
    z = float(np.float32(1e-35))
    return np.where((v >= -z) & (v <= z), 0.0, v)


STRUCT = ("split_feature", "threshold_in_bin", "decision_type", "left_child", "right_child",
          "leaf_count", "internal_count", "leaf_depth", "leaf_parent", "num_cat",
          "cat_boundaries", "cat_threshold")
VALUES = ("threshold", "leaf_value", "internal_value", "internal_weight", "leaf_weight")


def wide_bins_data(n, seed):
    """30 numerical features binned with max_bin 1023 / 4000 (some with NaN), 6
    categorical ones of 40 levels; a label driven by a few of each."""
    rng = np.random.default_rng(seed)
    n_num, n_cat = 30, 6
    Xn = rng.standard_normal((n_num, n))
    Xn[3, rng.random(n) < 0.05] = np.nan
    Xc = rng.integers(0, 40, (n_cat, n)).astype(np.float64)
    eff = rng.standard_normal((n_cat, 40))
    logit = Xn[0] - 0.7 * Xn[1] + np.nan_to_num(Xn[3]) * 0.5 + eff[0][Xc[0].astype(int)]
    y = (rng.random(n) < 1.0 / (1.0 + np.exp(-logit))).astype(np.float32)
    X = np.concatenate([Xn, Xc]).T
    cat = list(range(n_num, n_num + n_cat))
    ms = feature_mappers(X[:, :n_num], max_bin=1023, min_data_in_leaf=20)
    ms[0] = feature_mappers(X[:, :1], max_bin=4000, min_data_in_leaf=20)[0]
    ms += feature_mappers(X, categorical_features=cat, max_bin=255, min_data_in_leaf=20)[n_num:]
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint16)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f,
                         bin_type=m.bin_type) for f, m in enumerate(ms)]
    vals = np.concatenate([m.upper_bounds if m.bin_type == 0 else m.categories.astype(np.float64)
                           for m in ms])
    return X, y, ms, bins, meta, vals


def test_bin16_quantized_boosting_matches_oracle():
    n, iters, nl = 100_000, 3, 63
    X, y, ms, bins, meta, vals = wide_bins_data(n, 7)
    nbs = [m.num_bin for m in meta]
    assert max(nbs) > 2000 and sum(b > 256 for b in nbs) >= 20
    say(f"u16 bins n={n} max num_bin {max(nbs)}")
    init = oracle.boost_from_score(y)
    cfg = GainConfig.make(min_data_in_leaf=20)
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, vals)
        b.set_labels(y, init)
        trees = [b.train_iter_binary(i, cfg, nl, -1, 0.1, 4, True) for i in range(iters)]
        scores = b.scores()
    finally:
        b.close()
    oscores, otrees = oracle.train_binary(bins, meta, vals, y, cfg, nl, -1, iters, 0.1)
    used = set()
    for i, (t, o) in enumerate(zip(trees, otrees)):
        t = dict(t)
        if i == 0:
            t["leaf_value"] = _mrz(t["leaf_value"] + init)
            t["internal_value"] = _mrz(t["internal_value"] + init)
        assert t["num_leaves"] == o["num_leaves"], i
        for k in STRUCT:
            assert np.array_equal(np.asarray(t[k]), np.asarray(o[k])), (i, k)
        for k in VALUES:
            assert np.array_equal(bits(t[k]), bits(o[k])), (i, k)
        assert np.array_equal(np.asarray(t["split_gain"]), np.asarray(o["split_gain"])), i
        used.update(int(v) for v in o["threshold_in_bin"][:o["num_leaves"] - 1])
    assert max(used) > 255, "some split threshold lies past bin 255"
    assert np.array_equal(bits(scores), bits(oscores))


def test_bin16_f32_tree_and_layout():
    n = 60_000
    X, y, ms, bins, meta, vals = wide_bins_data(n, 8)
    rng = np.random.default_rng(9)
    g = rng.standard_normal(n).astype(np.float32)
    h = rng.uniform(0.05, 0.25, n).astype(np.float32)
    cfg = GainConfig.make(min_data_in_leaf=20)
    say(f"u16 bins f32 tree n={n}")
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, vals)
        b.upload_resident_grad_hess(g, h)
        t, lay = b.grow_tree_on_device_with_cfg(cfg, 127, -1)
    finally:
        b.close()
    o, olay = oracle.train_tree(bins, meta, vals, g, h, cfg, 127, -1)
    assert t["num_leaves"] == o["num_leaves"]
    for k in STRUCT:
        assert np.array_equal(np.asarray(t[k]), np.asarray(o[k])), k
    for k in ("leaf_value", "internal_value", "leaf_weight", "threshold"):
        np.testing.assert_allclose(t[k], o[k], rtol=1e-9, atol=1e-12, err_msg=k)
    assert np.array_equal(lay["indices"], olay["indices"])


def test_bin16_device_binning_matches_mappers():
    n = 50_000
    X, y, ms, bins, meta, vals = wide_bins_data(n, 10)
    say(f"u16 device binning n={n}")
    for col_major in (True, False):
        b = HipBackend(0)
        try:
            src = np.ascontiguousarray(X.T) if col_major else np.ascontiguousarray(X)
            b.upload_raw(src.astype(np.float32), ms, col_major=col_major)
            got = b.get_bins16()
        finally:
            b.close()
        want = np.stack([m.value_to_bin(X[:, j].astype(np.float32)) for j, m in enumerate(ms)])
        assert np.array_equal(got, want.astype(np.uint16)), col_major


def test_bin16_input_fitting_a_byte_trains_like_u8():
    from lightgbm_rs_amd.synth import config1_like
    n = 50_000
    bins, meta, ub, y = config1_like(n, seed=12)
    init = oracle.boost_from_score(y)
    cfg = GainConfig.make(min_data_in_leaf=20)
    runs = []
    for arr in (bins, bins.astype(np.uint16)):
        b = HipBackend(0)
        try:
            b.upload_resident_bins(arr, meta, ub)
            b.set_labels(y, init)
            runs.append(([b.train_iter_binary(i, cfg, 31, -1, 0.1, 4, True) for i in range(2)],
                         b.scores()))
        finally:
            b.close()
    assert np.array_equal(bits(runs[0][1]), bits(runs[1][1]))
    for t0, t1 in zip(runs[0][0], runs[1][0]):
        for k in STRUCT + VALUES:
            assert np.array_equal(np.asarray(t0[k]), np.asarray(t1[k])), k
