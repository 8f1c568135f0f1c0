"""Device feature contributions (TreeSHAP, `lgbm_hip_predict` kind CONTRIB) against
the real LightGBM binary's captures and the oracle.

Bars: f64 bits equal to the real binary's `pred_contrib` captures
(predict_modes/{numeric,categorical,multiclass}/contrib.txt); bits equal to the
oracle on seeded rows with NaNs for the committed model texts (numeric, categorical,
multiclass, missing-value handling) and for iteration slices; on 1M rows, which run
as two workspace chunks, the reference's invariant (per class the contributions and
the base sum to the raw score of the device predictor, within 1e-12) and the oracle's
bits on rows around the chunk boundary."""
import os

import numpy as np
import pytest

from lightgbm_rs_amd import HipBackend, HipError, Model
from oracle import predict as P
from tests import predict_modes as PM

pytestmark = pytest.mark.gpu
MT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_text")


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float64).view(np.uint64)


@pytest.mark.parametrize("name", ["numeric", "categorical", "multiclass"])
def test_device_contrib_matches_lightgbm(be, name):
    print("contrib capture", name, flush=True)
    text, X, ref = PM.contrib(name)
    got = be.predict(Model(text), X, "contrib")
    assert np.array_equal(bits(got), bits(ref))


@pytest.mark.parametrize("name", ["binary_spine", "cat_manyvsmany", "multiclass_spine",
                                  "na_missing", "rf_multi_bag", "forced_nested"])
def test_device_contrib_vs_oracle(be, name):
    print("contrib vs oracle", name, flush=True)
    text = open(os.path.join(MT, name + ".txt")).read()
    m, pm = Model(text), P.parse_model(text)
    rng = np.random.default_rng(3)
    X = rng.normal(scale=3.0, size=(300, pm["max_feature_idx"] + 1)).astype(np.float32)
    X[rng.random(X.shape) < 0.1] = np.nan
    X[rng.random(X.shape) < 0.1] = 0.0
    assert np.array_equal(bits(be.predict(m, X, "contrib")), bits(P.predict_contrib(pm, X)))
    total = pm["num_trees"] if "num_trees" in pm else len(pm["trees"]) // pm["num_tree_per_iteration"]
    if total >= 3:
        got = be.predict(m, X, "contrib", start_iteration=1, num_iteration=total - 2)
        ref = P.predict_contrib(pm, X, start_iteration=1, num_iteration=total - 2)
        assert np.array_equal(bits(got), bits(ref))


def test_device_contrib_large_two_chunks(be):
    print("contrib 1M rows", flush=True)
    text, X0, _ = PM.contrib("numeric")
    m, pm = Model(text), P.parse_model(text)
    rng = np.random.default_rng(9)
    lo, hi = np.nanmin(X0, axis=0), np.nanmax(X0, axis=0)
    X = rng.uniform(lo, hi, size=(1_000_000, X0.shape[1])).astype(np.float32)
    X[rng.random(X.shape) < 0.02] = np.nan
    got = be.predict(m, X, "contrib")
    nf = pm["max_feature_idx"] + 1
    raw = be.predict(m, X, "raw")
    np.testing.assert_allclose(got.reshape(len(X), -1, nf + 1).sum(axis=2), raw, rtol=0,
                               atol=1e-12)
    # a workspace chunk holds (256 MiB / bytes per row) rows rounded down to 256
    depth = max(P._max_depth(t) for t in pm["trees"])
    per_row = (depth + 1) * (depth + 2) // 2 * 28 + (depth + 1) * 24
    chunk = (256 << 20) // per_row // 256 * 256
    assert chunk < len(X)
    for r0 in (0, chunk - 150, len(X) - 300):
        sl = slice(r0, r0 + 300)
        assert np.array_equal(bits(got[sl]), bits(P.predict_contrib(pm, X[sl])))


def test_device_contrib_refuses_linear_trees(be):
    from tests.test_linear_cpu import load_case
    text, X, _ = load_case("reg_clean")
    with pytest.raises(HipError, match="linear"):
        be.predict(Model(text), X.astype(np.float32), "contrib")
