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
