"""Device prediction of linear-tree models (tree.rs:279-316) against the real
LightGBM 4.6.0 binary's linear goldens and the oracle.

Bars: raw predictions within the reference's ORACLE_TOL 1e-6 of C++
`booster.predict` on the f32-widened held-out rows (linear_parity.rs:160-173); equal
to the oracle's bits (same term order, f64, no fused multiply-add), on the goldens
and on a large seeded batch with NaN features, through both the LDS-staged rows
(up to 63 columns) and the direct rows."""
import numpy as np
import pytest

from lightgbm_rs_amd import HipBackend, Model
from oracle import predict as P
from tests.test_linear_cpu import CASES, load_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


@pytest.mark.parametrize("name", CASES)
def test_device_linear_predict_matches_lightgbm(be, name):
    print("linear golden", name, flush=True)
    text, X, pred = load_case(name)
    Xf = X.astype(np.float32)
    got = be.predict(Model(text), Xf, "raw")[:, 0]
    assert np.max(np.abs(got - pred)) <= 1e-6
    ref = P.predict(P.parse_model(text), Xf, kind="raw")[:, 0]
    assert np.array_equal(got.view(np.uint64), ref.view(np.uint64))


@pytest.mark.parametrize("extra_cols", [0, 70])
def test_device_linear_predict_large_vs_oracle(be, extra_cols):
    print("linear large batch, extra columns", extra_cols, flush=True)
    text, X, _ = load_case("reg_wide")
    rng = np.random.default_rng(11)
    n, c = 200_003, X.shape[1]
    Xl = rng.uniform(-0.2, 1.2, size=(n, c + extra_cols)).astype(np.float32)
    Xl[rng.random(Xl.shape) < 0.05] = np.nan
    m = Model(text)
    got = be.predict(m, Xl, "raw")[:, 0]
    ref = P.predict(P.parse_model(text), Xl, kind="raw")[:, 0]
    assert np.array_equal(got.view(np.uint64), ref.view(np.uint64))
    # the leaf kind is the plain tree walk, linear or not
    leaves = be.predict(m, Xl[:5000], "leaf")
    assert np.array_equal(leaves, P.predict(P.parse_model(text), Xl[:5000], kind="leaf"))
