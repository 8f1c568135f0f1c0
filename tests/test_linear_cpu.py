"""Linear trees (tree.rs:69-90, 279-316, 815-834, 1341-1412) on the CPU: the model
loader and writer of the C-ABI library, and the oracle's linear-leaf predictor, both
against the real LightGBM 4.6.0 binary's linear-tree goldens (tests/golden/linear/).

Pins: every model text round-trips byte-exact through the library (the C++ writer's
`leaf_features` / `leaf_coeff` layout, one extra space per leaf group); the oracle's
predictions on the f32-widened held-out rows match C++ `booster.predict` within the
reference's ORACLE_TOL 1e-6 (crates/oracle-harness/tests/linear_parity.rs:160-173,
which widens the rows from f32 the same way); a NaN feature of a leaf's model makes
the leaf answer its constant (`reg_nan_predict`), and a planted mistake in that rule
fails the pin."""
import glob
import os

import numpy as np
import pytest

from lightgbm_rs_amd import HipError, Model
from oracle import predict as P

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "linear")
CASES = sorted(os.path.basename(d) for d in glob.glob(os.path.join(GOLD, "reg_*")))


def load_case(name):
    d = os.path.join(GOLD, name)
    text = open(os.path.join(d, "model.txt")).read()
    X = np.loadtxt(os.path.join(d, "X_test.csv"), dtype=np.float64, ndmin=2)
    pred = np.loadtxt(os.path.join(d, "pred.csv"), dtype=np.float64)
    return text, X, pred


def test_cases_present():
    assert CASES == ["reg_bagging", "reg_clean", "reg_lambda", "reg_nan_predict",
                     "reg_one_round", "reg_wide"]


@pytest.mark.parametrize("name", CASES)
def test_linear_model_text_round_trips_byte_exact(name):
    text, _, _ = load_case(name)
    assert "is_linear=1" in text
    assert Model(text).to_text() == text


@pytest.mark.parametrize("name", CASES)
def test_oracle_linear_predict_matches_lightgbm(name):
    text, X, pred = load_case(name)
    got = P.predict(P.parse_model(text), X.astype(np.float32), kind="raw")[:, 0]
    assert np.max(np.abs(got - pred)) <= 1e-6


def test_linear_models_have_terms_and_nan_rows():
    # the goldens cover leaves with linear terms and rows whose terms are NaN
    text, X, _ = load_case("reg_nan_predict")
    m = P.parse_model(text)
    assert any(len(f) for t in m["trees"] for (_, f, _) in t.get("linear", []))
    assert np.isnan(X).any()


def test_planted_nan_rule_mistake_fails_the_pin():
    text, X, pred = load_case("reg_nan_predict")
    m = P.parse_model(text)
    Xf = X.astype(np.float32)
    ok = P.predict(m, Xf, kind="raw")[:, 0]
    assert np.max(np.abs(ok - pred)) <= 1e-6
    # a NaN term treated as 0 (the plain numeric decision's missing rule) instead of
    # falling back to the leaf's constant
    bad = P.predict(m, np.nan_to_num(Xf, nan=0.0), kind="raw")[:, 0]
    rows = np.isnan(X).any(axis=1)
    assert np.max(np.abs(bad[rows] - pred[rows])) > 1e-6


def _tree_edit(text, key, new):
    head, body = text.split("\nTree=0\n", 1)
    lines = body.split("\n")
    for i, line in enumerate(lines):
        if line.startswith(key + "="):
            lines[i] = key + "=" + new
            break
    else:
        raise AssertionError(key)
    return head + "\nTree=0\n" + "\n".join(lines)


@pytest.mark.parametrize("key,new,needle", [
    ("leaf_const", "1 2", "leaf_const length"),
    ("num_features", "-1 0 0 0 0 0 0", "negative"),
    ("num_features", "1 0 0 0 0 0 0", "leaf_features length"),
])
def test_malformed_linear_blocks_are_rejected(key, new, needle):
    text, _, _ = load_case("reg_clean")
    with pytest.raises(HipError, match=needle):
        Model(_tree_edit(text, key, new))


def test_linear_feature_out_of_range_is_rejected():
    text, _, _ = load_case("reg_nan_predict")
    m = P.parse_model(text)
    t0 = next(i for i, t in enumerate(m["trees"])
              if any(len(f) for (_, f, _) in t.get("linear", [])))
    blocks = text.split("\nTree=")
    blk = blocks[t0 + 1]
    line = next(ln for ln in blk.split("\n") if ln.startswith("leaf_features="))
    toks = line[len("leaf_features="):].split(" ")
    j = next(i for i, tk in enumerate(toks) if tk)
    toks[j] = "99"
    blocks[t0 + 1] = blk.replace(line, "leaf_features=" + " ".join(toks))
    with pytest.raises(HipError, match="leaf_features entry out of range"):
        Model("\nTree=".join(blocks))
