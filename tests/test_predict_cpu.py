"""Model text + batch prediction, CPU side: the oracle predictor pinned to the
reference's prediction goldens, hand-derived missing-value routing, and the
library's host-only model loader (no GPU needed)."""
import math
import os

import numpy as np
import pytest

from lightgbm_rs_amd import HipError, Model
from oracle import predict as P

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "predict")
CORPORA = ["binary", "categorical", "regression", "multiclass", "subrange"]


def corpus(name):
    text = open(os.path.join(GOLD, name + "_model.txt")).read()
    return text, np.load(os.path.join(GOLD, name + ".npz"))


def bits(a):
    return np.ascontiguousarray(a).view(np.uint64)


@pytest.mark.parametrize("name", CORPORA)
def test_oracle_matches_reference_goldens(name):
    text, d = corpus(name)
    m = P.parse_model(text)
    assert np.array_equal(bits(P.predict(m, d["X"], kind="raw")), bits(d["raw"]))
    assert np.array_equal(bits(P.predict(m, d["X"], kind="transformed")), bits(d["transformed"]))
    assert np.array_equal(P.predict(m, d["X"], kind="leaf"), d["leaf"])


def test_oracle_iteration_slices_match_reference():
    text, d = corpus("subrange")
    m = P.parse_model(text)
    for s, n, v in zip(d["slice_start"], d["slice_num"], d["slice_raw"]):
        got = P.predict(m, d["X"], start_iteration=int(s), num_iteration=int(n), kind="raw")[:, 0]
        assert np.array_equal(bits(got), bits(v)), (s, n)


# One split on feature 0 at 0.5 (leaf 0 left, leaf 1 right), the decision_type
# varied: bit 1 default-left, bits 2-3 missing type (1 zero, 2 NaN).
MISSING_MODEL = """tree
version=v4
num_class=1
num_tree_per_iteration=1
label_index=0
max_feature_idx=1
objective=regression
feature_names=a b
feature_infos=[0:1] [0:1]
tree_sizes=0

Tree=0
num_leaves=2
num_cat=0
split_feature=0
split_gain=1
threshold=0.5
decision_type={dt}
left_child=-1
right_child=-2
leaf_value=-1 1
leaf_weight=1 1
leaf_count=1 1
internal_value=0
internal_weight=2
internal_count=2
is_linear=0
shrinkage=1


end of trees
"""


@pytest.mark.parametrize("dt,expected", [
    # rows: NaN, 0, 1e-36, -1e-36, 0.3, 0.7, -2
    (0, [0, 0, 0, 0, 0, 1, 0]),  # no missing type: NaN -> 0.0 -> left (<= 0.5)
    (2, [0, 0, 0, 0, 0, 1, 0]),  # default-left alone changes nothing
    (4, [1, 1, 1, 1, 0, 1, 0]),  # zero missing, default right: NaN -> 0 -> zero -> right
    (6, [0, 0, 0, 0, 0, 1, 0]),  # zero missing, default left
    (8, [1, 0, 0, 0, 0, 1, 0]),  # NaN missing, default right: only NaN is missing
    (10, [0, 0, 0, 0, 0, 1, 0]),  # NaN missing, default left
])
def test_missing_value_routing(dt, expected):
    m = P.parse_model(MISSING_MODEL.format(dt=dt))
    X = np.array([[math.nan, 0], [0, 0], [1e-36, 0], [-1e-36, 0], [0.3, 0], [0.7, 0], [-2, 0]],
                 np.float32)
    assert P.predict(m, X, kind="leaf")[:, 0].tolist() == expected


@pytest.mark.parametrize("name", CORPORA)
def test_library_loads_reference_models(name):
    text, d = corpus(name)
    ref = P.parse_model(text)
    m = Model(text)
    assert m.num_trees == len(ref["trees"])
    assert m.num_class == ref["num_class"]
    assert m.num_tree_per_iteration == ref["num_tree_per_iteration"]
    assert m.max_feature_idx == ref["max_feature_idx"]
    assert m.num_iterations == len(ref["trees"]) // ref["num_tree_per_iteration"]
    m.close()


@pytest.mark.parametrize("edit,needle", [
    (lambda t: t.replace("objective=regression", "objective=lambdarank"), "not supported"),
    (lambda t: t.replace("is_linear=0", "is_linear=1"), "linear"),
    (lambda t: t.replace("right_child=-2", "right_child=-3"), "out of range"),
    (lambda t: t.replace("right_child=-2", "right_child=0"), "out of range"),
    (lambda t: t.replace("split_feature=0", "split_feature=2"), "split_feature"),
    (lambda t: t.replace("leaf_value=-1 1", "leaf_value=-1"), "leaf_value"),
    (lambda t: t.replace("threshold=0.5\n", ""), "threshold"),
    (lambda t: t.replace("num_class=1\n", ""), "num_class"),
    (lambda t: t.replace("decision_type={dt}", "decision_type=1"), "categorical"),
])
def test_library_rejects_malformed_models(edit, needle):
    text = edit(MISSING_MODEL).replace("{dt}", "0")
    with pytest.raises(HipError) as e:
        Model(text)
    assert needle in str(e.value)


@pytest.mark.parametrize("name", ["numeric", "multiclass"])
def test_oracle_early_stop_matches_reference_captures(name):
    """Prediction early stopping (predict_parity.rs:160-226): every (freq, margin)
    cell's frozen raw scores; the regression model ignores the request (accurate
    prediction) and the multiclass model stops at its margin."""
    from tests import predict_modes as PM
    text, X, cells = PM.corpus(name)
    m = P.parse_model(text)
    full = P.predict(m, X, kind="raw")
    stopped = False
    for freq, margin, exp in cells:
        raw, iters = P.predict_early_stop(m, X, freq, margin)
        assert np.array_equal(bits(raw), bits(exp)), (freq, margin)
        stopped |= bool(np.any(iters < len(m["trees"]) // m["num_tree_per_iteration"]))
    assert stopped == (name == "multiclass")
    if name == "numeric":
        assert np.array_equal(bits(cells[0][2]), bits(full))
