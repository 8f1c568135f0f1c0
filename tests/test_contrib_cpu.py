"""Feature contributions (TreeSHAP, tree.rs:336-583; predict.rs:607-697) in the
oracle, pinned three ways:
- the real LightGBM binary's `predict(pred_contrib=True)` captures
  (oracle-harness/tests/fixtures/predict_modes/{numeric,categorical,multiclass}/
  contrib.txt, f64 bits): bit-exact;
- the definition: on small random trees (repeated features, NaN inputs, chains) the
  Shapley values computed by brute force over every feature subset, with the value
  of a subset the cover-weighted expectation of the tree given those features;
- the reference's invariant: per class, the contributions and the base sum to the
  raw score.
A planted mistake (the base as the plain mean of the leaves instead of the
cover-weighted one) fails the capture pin."""
import itertools
import math

import numpy as np
import pytest

from oracle import predict as P
from tests import predict_modes as PM

CORPORA = ["numeric", "categorical", "multiclass"]


@pytest.mark.parametrize("name", CORPORA)
def test_oracle_contrib_matches_lightgbm_bits(name):
    text, X, ref = PM.contrib(name)
    got = P.predict_contrib(P.parse_model(text), X)
    assert got.shape == ref.shape
    assert np.array_equal(got.view(np.uint64), ref.view(np.uint64))


@pytest.mark.parametrize("name", CORPORA)
def test_contrib_sums_to_raw_score(name):
    text, X, _ = PM.contrib(name)
    m = P.parse_model(text)
    ntpi, nf = m["num_tree_per_iteration"], m["max_feature_idx"] + 1
    c = P.predict_contrib(m, X).reshape(len(X), ntpi, nf + 1)
    np.testing.assert_allclose(c.sum(axis=2), P.predict(m, X, kind="raw"), rtol=0, atol=1e-12)


def random_tree(rng, num_leaves, n_feat, chain=False):
    """A random tree of `num_leaves` leaves over `n_feat` features (features repeat
    along paths), with leaf counts drawn at random and internal counts their sums."""
    left, right, feat = [], [], []
    where = {0: None}  # leaf -> (node, side) of the slot that holds it
    for s in range(num_leaves - 1):
        lid = max(where) if chain else int(rng.choice(sorted(where)))
        slot = where.pop(lid)
        n = len(left)
        left.append(~lid)
        right.append(~(s + 1))
        feat.append(int(rng.integers(n_feat)))
        if slot is not None:
            (left if slot[1] == 0 else right)[slot[0]] = n
        where[lid], where[s + 1] = (n, 0), (n, 1)
    lc = rng.integers(1, 40, size=num_leaves)
    ic = np.zeros(max(num_leaves - 1, 0), np.int64)

    def count(c):
        if c < 0:
            return int(lc[~c])
        ic[c] = count(left[c]) + count(right[c])
        return int(ic[c])

    t = {"num_leaves": num_leaves, "num_cat": 0, "leaf_value": rng.normal(size=num_leaves),
         "leaf_count": lc}
    if num_leaves > 1:
        count(0)
        t.update(split_feature=np.array(feat), threshold=rng.normal(size=num_leaves - 1),
                 decision_type=np.full(num_leaves - 1, 2 | (2 << 2)),  # NaN goes left
                 left_child=np.array(left), right_child=np.array(right), internal_count=ic)
    return t


def _value(t, x, S, node=0):
    """E[tree | the features in S fixed to x], splits on other features averaged by cover."""
    if t["num_leaves"] == 1:
        return float(t["leaf_value"][0])
    if node < 0:
        return float(t["leaf_value"][~node])
    f = int(t["split_feature"][node])
    if f in S:
        nxt = int(P._decide(t, np.array([node]), np.array([x[f]], dtype=np.float64))[0])
        return _value(t, x, S, nxt)
    kids = [int(t["left_child"][node]), int(t["right_child"][node])]
    return sum(float(P._count(t, k)) * _value(t, x, S, k) for k in kids) / P._count(t, node)


def brute_force_shap(t, x, n_feat):
    phi = np.zeros(n_feat + 1)
    for i in range(n_feat):
        others = [j for j in range(n_feat) if j != i]
        for size in range(n_feat):
            w = math.factorial(size) * math.factorial(n_feat - size - 1) / math.factorial(n_feat)
            for S in itertools.combinations(others, size):
                phi[i] += w * (_value(t, x, set(S) | {i}) - _value(t, x, set(S)))
    phi[n_feat] = _value(t, x, set())
    return phi


@pytest.mark.parametrize("seed,num_leaves,n_feat,chain", [
    (1, 1, 3, False), (2, 2, 1, False), (3, 7, 3, False), (4, 15, 4, False), (5, 9, 2, True),
    (6, 20, 4, False), (7, 12, 3, True)])
def test_oracle_contrib_equals_brute_force_shapley(seed, num_leaves, n_feat, chain):
    rng = np.random.default_rng(seed)
    t = random_tree(rng, num_leaves, n_feat, chain)
    m = {"num_tree_per_iteration": 1, "max_feature_idx": n_feat - 1, "trees": [t]}
    X = rng.normal(size=(6, n_feat)).astype(np.float32)
    X[0, 0] = np.nan
    got = P.predict_contrib(m, X)
    for r in range(len(X)):
        ref = brute_force_shap(t, X[r].astype(np.float64), n_feat)
        np.testing.assert_allclose(got[r], ref, rtol=0, atol=1e-12)


def test_planted_base_mistake_fails_the_pin(monkeypatch):
    text, X, ref = PM.contrib("numeric")
    m = P.parse_model(text)
    monkeypatch.setattr(P, "expected_value", lambda t: float(np.mean(t["leaf_value"])))
    got = P.predict_contrib(m, X)
    assert not np.array_equal(got.view(np.uint64), ref.view(np.uint64))


def test_oracle_contrib_refuses_linear_trees():
    from tests.test_linear_cpu import load_case
    text, X, _ = load_case("reg_clean")
    with pytest.raises(ValueError, match="linear"):
        P.predict_contrib(P.parse_model(text), X[:2])
