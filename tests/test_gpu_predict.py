"""Device batch prediction vs the reference's prediction goldens and the oracle.

Bar: raw scores bit-exact (the same f64 additions in the same order), leaf indices
exact; transformed outputs within 1e-14 relative (the device's exp/log1p may differ
from the host libm's in the last bits)."""
import math
import os

import numpy as np
import pytest

from lightgbm_rs_amd import HipBackend, HipError, Model
from oracle import predict as P

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "predict")
CORPORA = ["binary", "categorical", "regression", "multiclass", "subrange"]


def corpus(name):
    text = open(os.path.join(GOLD, name + "_model.txt")).read()
    return text, np.load(os.path.join(GOLD, name + ".npz"))


def bits(a):
    return np.ascontiguousarray(a).view(np.uint64)


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


@pytest.mark.parametrize("name", CORPORA)
def test_predict_matches_reference_goldens(be, name):
    print(f"predict goldens {name}", flush=True)
    text, d = corpus(name)
    m = Model(text)
    assert np.array_equal(bits(be.predict(m, d["X"], "raw")), bits(d["raw"]))
    assert np.array_equal(be.predict(m, d["X"], "leaf"), d["leaf"])
    np.testing.assert_allclose(be.predict(m, d["X"], "transformed"), d["transformed"], rtol=1e-14,
                               atol=0)


def test_predict_iteration_slices(be):
    text, d = corpus("subrange")
    m = Model(text)
    for s, n, v in zip(d["slice_start"], d["slice_num"], d["slice_raw"]):
        got = be.predict(m, d["X"], "raw", int(s), int(n))[:, 0]
        assert np.array_equal(bits(got), bits(v)), (s, n)
    full = be.predict(m, d["X"], "leaf")
    for s, n in [(0, 3), (4, -1), (9, 5), (12, 1), (-3, 2)]:
        got = be.predict(m, d["X"], "leaf", s, n)
        start = min(max(s, 0), 10)
        num = min(n, 10 - start) if n > 0 else 10 - start
        assert np.array_equal(got, full[:, start:start + num]), (s, n)


def _edge_rows(rng, X, frac=0.1):
    """Rows of X with NaN, exact zeros, tiny magnitudes and negative categories."""
    X = X.copy()
    n, f = X.shape
    for v in (np.nan, 0.0, 1e-36, -1e-36, -1.0, 3.0, 7.9, 1e30):
        mask = rng.random((n, f)) < frac / 8
        X[mask] = v
    return X


@pytest.mark.parametrize("name", CORPORA)
def test_predict_edge_values_vs_oracle(be, name):
    text, d = corpus(name)
    m, om = Model(text), P.parse_model(text)
    rng = np.random.default_rng(7)
    X = _edge_rows(rng, np.tile(d["X"], (4, 1)))
    assert np.array_equal(bits(be.predict(m, X, "raw")), bits(P.predict(om, X, kind="raw")))
    assert np.array_equal(be.predict(m, X, "leaf"), P.predict(om, X, kind="leaf"))


def test_predict_large_batch_vs_oracle(be):
    text, d = corpus("multiclass")
    m, om = Model(text), P.parse_model(text)
    rng = np.random.default_rng(3)
    n = 300_000
    X = (d["X"][rng.integers(0, len(d["X"]), n)] + rng.normal(0, 0.05, (n, 28))).astype(np.float32)
    got = be.predict(m, X, "raw")
    exp = P.predict(om, X, kind="raw")
    assert np.array_equal(bits(got), bits(exp))


def test_predict_device_buffers(be):
    """Device-resident input and output through the HIP runtime the library uses."""
    import ctypes as C
    hip = C.CDLL("/opt/rocm/lib/libamdhip64.so.7")
    text, d = corpus("binary")
    m = Model(text)
    X = np.ascontiguousarray(d["X"])
    dx, dout = C.c_void_p(), C.c_void_p()
    assert hip.hipMalloc(C.byref(dx), C.c_size_t(X.nbytes)) == 0
    assert hip.hipMalloc(C.byref(dout), C.c_size_t(len(X) * 8)) == 0
    try:
        assert hip.hipMemcpy(dx, X.ctypes.data_as(C.c_void_p), C.c_size_t(X.nbytes), 1) == 0
        be.predict_device(m, dx.value, X.shape[0], X.shape[1], dout.value, "raw")
        out = np.zeros((len(X), 1), np.float64)
        assert hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), dout, C.c_size_t(out.nbytes), 2) == 0
        assert np.array_equal(bits(out), bits(d["raw"]))
    finally:
        hip.hipFree(dx)
        hip.hipFree(dout)


def test_predict_errors(be):
    text, d = corpus("binary")
    m = Model(text)
    with pytest.raises(HipError) as e:
        be.predict(m, d["X"][:, :20], "raw")
    assert e.value.code == -1  # LENGTH_MISMATCH: fewer columns than max_feature_idx + 1
    assert be.predict(m, d["X"][:0], "raw").shape == (0, 1)


@pytest.mark.parametrize("name", ["rf_multi_bag", "rf_single_bag"])
def test_predict_average_output_vs_oracle(be, name):
    """Random-forest models (average_output): transformed divides the raw sum by the
    iteration count before ConvertOutput (predict.rs:338-349)."""
    text = open(os.path.join(os.path.dirname(GOLD), "model_text", name + ".txt")).read()
    m, om = Model(text), P.parse_model(text)
    X = np.random.default_rng(5).normal(size=(4096, m.max_feature_idx + 1)).astype(np.float32)
    assert np.array_equal(bits(be.predict(m, X, "raw")), bits(P.predict(om, X, kind="raw")))
    np.testing.assert_allclose(be.predict(m, X, "transformed"),
                               P.predict(om, X, kind="transformed"), rtol=1e-14, atol=0)


def test_transformed_needs_objective(be):
    text = open(os.path.join(os.path.dirname(GOLD), "model_text", "custom_no_objective.txt")).read()
    m = Model(text)
    X = np.zeros((3, m.max_feature_idx + 1), np.float32)
    be.predict(m, X, "raw")
    with pytest.raises(HipError) as e:
        be.predict(m, X, "transformed")
    assert "objective" in str(e.value)


def _binned_table(n, seed, max_bin=63):
    """float32 features with their quantile bins (bin b <=> ub[b-1] < x <= ub[b])."""
    from lightgbm_rs_amd.synth import _meta_for
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, 12)).astype(np.float32)
    X[:, 3] = np.round(X[:, 3] * 2)  # a few-valued column
    w = rng.standard_normal(12).astype(np.float32)
    y = (rng.random(n) < 1 / (1 + np.exp(-(X @ w)))).astype(np.float32)
    bins = np.zeros((12, n), np.uint8)
    ub, nbs = [], []
    for f in range(12):
        qs = np.unique(np.quantile(X[:, f], np.linspace(0, 1, max_bin + 1)[1:-1]).astype(np.float32))
        bins[f] = np.searchsorted(qs, X[:, f], side="left")
        nbs.append(len(qs) + 1)
        ub.extend([float(q) for q in qs] + [np.inf])
    return X, bins, _meta_for(nbs), np.array(ub), y


@pytest.mark.parametrize("quant", [4, 0])
def test_trained_model_text_predicts_training_scores(be, quant):
    """Trees grown by the resident boosting loop, assembled into a model (the first
    tree carrying the init score), written as model text and read back: the device
    predictor reproduces the training scores bit for bit."""
    from lightgbm_rs_amd import GainConfig, binary_boost_from_score
    print(f"trained model predict quant={quant}", flush=True)
    X, bins, meta, ub, y = _binned_table(30_000, seed=41)
    init = binary_boost_from_score(y)
    be.upload_resident_bins(bins, meta, ub)
    be.set_labels(y, init)
    cfg = GainConfig.make(min_data_in_leaf=20)
    m = Model.create(num_class=1, max_feature_idx=11, objective="binary sigmoid:1")
    for i in range(6):
        t = be.train_iter_binary(i, cfg, 31, -1, 0.1, quant, quant > 0)
        assert np.all(t["internal_weight"] > 0)
        m.add_tree(t, shrinkage=0.1, bias=init if i == 0 else 0.0)
    scores = be.scores()
    text = m.to_text()
    back = Model(text)
    assert back.to_text() == text
    got = be.predict(back, X, "raw")[:, 0]
    assert np.array_equal(bits(got), bits(scores))
    assert np.array_equal(bits(P.predict(P.parse_model(text), X, kind="raw")[:, 0]), bits(scores))


@pytest.mark.parametrize("name", ["numeric", "multiclass"])
def test_device_early_stop_matches_reference_captures(be, name):
    from tests import predict_modes as PM
    text, X, cells = PM.corpus(name)
    m, om = Model(text), P.parse_model(text)
    for freq, margin, exp in cells:
        raw, iters = be.predict_early_stop(m, X, freq, margin)
        assert np.array_equal(bits(raw), bits(exp)), (freq, margin)
        _, oiters = P.predict_early_stop(om, X, freq, margin)
        assert np.array_equal(iters, oiters), (freq, margin)


def test_device_early_stop_vs_oracle_large(be):
    """More rows, several margins and an iteration slice, against the oracle."""
    text, d = corpus("multiclass")
    m, om = Model(text), P.parse_model(text)
    rng = np.random.default_rng(8)
    X = (d["X"][rng.integers(0, len(d["X"]), 3000)] + rng.normal(0, 0.1, (3000, 28))).astype(np.float32)
    for freq, margin, s, n in [(1, 0.5, 0, -1), (3, 2.0, 0, -1), (2, 1.0, 2, 6), (5, 0.0, 0, -1)]:
        raw, iters = be.predict_early_stop(m, X, freq, margin, s, n)
        oraw, oiters = P.predict_early_stop(om, X, freq, margin, s, n)
        assert np.array_equal(bits(raw), bits(oraw)), (freq, margin, s, n)
        assert np.array_equal(iters, oiters), (freq, margin, s, n)
