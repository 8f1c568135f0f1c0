"""Device binning (lgbm_hip_upload_raw*): raw feature matrices binned on the GPU into
the resident records, checked bin for bin against the reference's ValueToBin goldens
and the oracle, then trained on end to end.  Bar: exact."""
import ctypes as C

import numpy as np
import pytest

from tests import binning_fixtures as BF
from lightgbm_rs_amd import (BinMapper, GainConfig, HipBackend, HipError, Model,
                             binary_boost_from_score, feature_mappers)
from oracle import binning as OB

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


def _oracle(mappers, X):
    return np.stack([OB.value_to_bin_numeric(X[:, f], m.upper_bounds, m.missing_type)
                     for f, m in enumerate(mappers)])


@pytest.mark.parametrize("ds", BF.datasets("example_dataset_binning"),
                         ids=lambda d: d["params"]["name"])
def test_device_bins_match_reference_goldens(be, ds):
    print(f"device binning {ds['params']['name']}", flush=True)
    X = BF.examples()[ds["params"]["name"].split(".")[0]]
    ms = [BinMapper.from_column(X[:, f], max_bin=255, min_data_in_bin=3, min_data_in_leaf=20,
                                bin_construct_sample_cnt=100000,
                                data_random_seed=int(ds["params"]["seed"]))
          for f in range(X.shape[1])]
    be.upload_raw(X, ms)
    got = be.get_bins()
    for f in range(X.shape[1]):
        assert np.array_equal(got[f], ds["assign"][f]), f


def _table(n, F, seed):
    rng = np.random.default_rng(seed)
    X = rng.normal(size=(n, F))
    X[:, 1] = np.round(X[:, 1] * 3)                        # few distinct values
    X[rng.random((n, F)) < 0.03] = np.nan                  # missing
    X[:, 2] = np.where(rng.random(n) < 0.6, 0.0, X[:, 2])  # mostly zeros
    X[:, 3] = -np.abs(X[:, 3])                             # negative only
    X[:5, 4] = [np.inf, -np.inf, -0.0, 1e-36, -1e-36]
    return X


@pytest.mark.parametrize("dtype,col_major", [(np.float64, False), (np.float32, False),
                                             (np.float64, True), (np.float32, True)])
def test_device_bins_match_oracle(be, dtype, col_major):
    n, F = 300_000, 13
    print(f"device binning dtype={np.dtype(dtype).name} col_major={col_major}", flush=True)
    X = _table(n, F, seed=5).astype(dtype)
    ms = feature_mappers(X, max_bin=63, zero_as_missing=False)
    be.upload_raw(X.T.copy() if col_major else X, ms, col_major=col_major)
    assert np.array_equal(be.get_bins(), _oracle(ms, X.astype(np.float64)))


def test_device_bins_zero_as_missing_and_max_bin_255(be):
    X = _table(200_000, 7, seed=8)
    ms = feature_mappers(X, max_bin=255, zero_as_missing=True)
    assert max(m.num_bin for m in ms) > 200
    be.upload_raw(X, ms)
    assert np.array_equal(be.get_bins(), _oracle(ms, X))


def test_device_bins_from_device_memory(be):
    hip = C.CDLL("/opt/rocm/lib/libamdhip64.so.7")
    X = np.ascontiguousarray(_table(50_000, 9, seed=9))
    ms = feature_mappers(X)
    d = C.c_void_p()
    assert hip.hipMalloc(C.byref(d), C.c_size_t(X.nbytes)) == 0
    try:
        assert hip.hipMemcpy(d, X.ctypes.data_as(C.c_void_p), C.c_size_t(X.nbytes), 1) == 0
        be.upload_raw_device(d.value, np.float64, X.shape[0], X.shape[1], ms)
        assert np.array_equal(be.get_bins(), _oracle(ms, X))
    finally:
        hip.hipFree(d)


def test_categorical_columns_bin_like_the_mapper(be):
    """Categorical columns on the device: ValueToBin of the categorical mapper (the
    sorted (category, bin) table), NaN / negative / unseen categories to bin 0."""
    rng = np.random.default_rng(1)
    n = 50_000
    X = np.empty((n, 3), np.float64)
    X[:, 0] = rng.standard_normal(n)
    X[:, 1] = rng.integers(0, 40, n)
    X[:, 2] = rng.integers(0, 7, n)
    ms = feature_mappers(X[:40_000], categorical_features=[1, 2], max_bin=255)
    X[::97, 1] = np.nan
    X[::89, 1] = -3.0
    X[::83, 2] = 1000.0  # unseen by the mapper
    X[::79, 2] = 2.7     # truncates to category 2
    be.upload_raw(X, ms)
    got = be.get_bins()
    for f, m in enumerate(ms):
        assert np.array_equal(got[f], m.value_to_bin(X[:, f]).astype(np.uint8)), f
    unseen = np.arange(0, n, 83)
    unseen = unseen[unseen % 79 != 0]  # rows not overwritten with 2.7
    assert (got[1][::97] == 0).all() and (got[2][unseen] == 0).all()


def test_raw_to_model_predicts_training_scores(be):
    """Raw features -> device bins -> resident boosting -> model text -> device
    prediction on the same raw features reproduces the training scores bit for bit
    (the bin upper bounds are the split thresholds)."""
    n = 40_000
    X = _table(n, 10, seed=17).astype(np.float32).astype(np.float64)  # the predictor reads f32
    rng = np.random.default_rng(3)
    logit = np.nan_to_num(X[:, 0]) - 0.5 * np.nan_to_num(X[:, 5]) + 0.3 * np.nan_to_num(X[:, 1])
    y = (rng.random(n) < 1 / (1 + np.exp(-logit))).astype(np.float32)
    ms = feature_mappers(X, max_bin=63)
    be.upload_raw(X, ms)
    init = binary_boost_from_score(y)
    be.set_labels(y, init)
    cfg = GainConfig.make(min_data_in_leaf=20)
    infos = " ".join(f"[{np.nanmin(X[:, f]):g}:{np.nanmax(X[:, f]):g}]" for f in range(10))
    m = Model.create(num_class=1, max_feature_idx=9, objective="binary sigmoid:1",
                     feature_infos=infos)
    for i in range(5):
        t = be.train_iter_binary(i, cfg, 31, -1, 0.1)
        m.add_tree(t, shrinkage=0.1, bias=init if i == 0 else 0.0)
    back = Model(m.to_text())
    got = be.predict(back, X.astype(np.float32), "raw")[:, 0]
    assert np.array_equal(got.view(np.uint64), be.scores().view(np.uint64))
