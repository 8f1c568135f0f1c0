"""Model text writer, CPU side (no GPU needed).

The pins: every committed model text of the reference's tests (written by the real
LightGBM 4.6 binary) loads and is written back byte for byte; a model assembled
from grown trees is checked against Python's own printf formatting (`%.17g` /
`%g`), independently recomputed tree_sizes and split-count importances, and the
bias / shrinkage rules of Tree::add_bias / Tree::shrinkage
(crates/lgbm-model/src/tree.rs:1074-1168)."""
import glob
import math
import os

import numpy as np
import pytest

from lightgbm_rs_amd import HipError, Model
from oracle import predict as P

HERE = os.path.dirname(os.path.abspath(__file__))
TEXTS = sorted(glob.glob(os.path.join(HERE, "golden", "model_text", "*.txt")) +
               glob.glob(os.path.join(HERE, "golden", "predict", "*_model.txt")))


def _id(p):
    return os.path.basename(p)[:-4]


@pytest.mark.parametrize("path", TEXTS, ids=_id)
def test_reference_model_texts_round_trip_byte_exact(path):
    text = open(path, newline="").read()
    m = Model(text)
    assert m.to_text() == text
    ref = P.parse_model(text)
    assert m.num_trees == len(ref["trees"])


def test_fixture_coverage():
    """The fixtures exercise the envelope and block forms the writer has."""
    texts = {_id(p): open(p).read() for p in TEXTS}
    assert any("average_output\n" in t for t in texts.values())
    assert any("monotone_constraints=" in t for t in texts.values())
    assert any("\ncat_threshold=" in t for t in texts.values())
    assert any("\nleaf_weight=\n" in t for t in texts.values())
    assert any("\nobjective=" not in t for t in texts.values())
    assert any("\nparameters:\n" in t for t in texts.values())


def _tree(rng, num_leaves, n_feat):
    """A random well-formed tree in the layout Tree::split grows (tree.rs:614-700)."""
    ni = num_leaves - 1
    left, right = [~0], [~1]
    parent_of_leaf = {0: (0, 0), 1: (0, 1)}
    for node in range(1, ni):
        leaf = int(rng.integers(0, node + 1))
        p, side = parent_of_leaf[leaf]
        (left if side == 0 else right)[p] = node
        left.append(~leaf)
        right.append(~(node + 1))
        parent_of_leaf[leaf] = (node, 0)
        parent_of_leaf[node + 1] = (node, 1)
    return {
        "num_leaves": num_leaves,
        "split_feature": rng.integers(0, n_feat, ni).astype(np.int32),
        "threshold": rng.normal(size=ni) * 10.0 ** rng.integers(-5, 6, ni),
        "split_gain": np.abs(rng.normal(size=ni)).astype(np.float32) * 100,
        "decision_type": np.full(ni, 2, np.int8),
        "left_child": np.array(left, np.int32),
        "right_child": np.array(right, np.int32),
        "internal_value": rng.normal(size=ni),
        "internal_count": rng.integers(1, 1000, ni).astype(np.int32),
        "leaf_value": rng.normal(size=num_leaves) * 10.0 ** rng.integers(-8, 3, num_leaves),
        "leaf_weight": np.abs(rng.normal(size=num_leaves)) * 50,
        "leaf_count": rng.integers(1, 1000, num_leaves).astype(np.int32),
    }


def _field(block, key):
    for line in block.split("\n"):
        if line.startswith(key + "="):
            return line[len(key) + 1:]
    raise KeyError(key)


def test_writer_fields_formats_and_envelope():
    rng = np.random.default_rng(11)
    n_feat = 6
    m = Model.create(num_class=1, max_feature_idx=n_feat - 1, objective="binary sigmoid:1")
    trees = [_tree(rng, nl, n_feat) for nl in (7, 2, 31, 5)]
    bias = 0.37
    for i, t in enumerate(trees):
        # the first tree carries the init score: AddBias forces its shrinkage to 1
        m.add_tree(t, shrinkage=0.1, bias=bias if i == 0 else 0.0)
    text = m.to_text()
    head, rest = text.split("\n\n", 1)
    assert head.split("\n")[:8] == [
        "tree", "version=v4", "num_class=1", "num_tree_per_iteration=1", "label_index=0",
        "max_feature_idx=5", "objective=binary sigmoid:1",
        "feature_names=" + " ".join(f"Column_{f}" for f in range(n_feat))]
    assert _field(head, "feature_infos") == " ".join(["none"] * n_feat)
    body, tail = rest.split("end of trees\n", 1)
    blocks = ["Tree=" + b for b in body.split("Tree=")[1:]]
    assert [int(x) for x in _field(head, "tree_sizes").split()] == [len(b.encode()) for b in blocks]
    for i, (t, b) in enumerate(zip(trees, blocks)):
        assert b.startswith(f"Tree={i}\nnum_leaves={t['num_leaves']}\nnum_cat=0\n")
        assert b.endswith("is_linear=0\nshrinkage=%g\n\n\n" % (1.0 if i == 0 else 0.1))
        add = bias if i == 0 else 0.0
        lv = [v + add for v in t["leaf_value"]]
        lv = [0.0 if abs(v) <= float(np.float32(1e-35)) else v for v in lv]
        iv = [v + add for v in t["internal_value"]]
        assert _field(b, "leaf_value") == " ".join("%.17g" % v for v in lv)
        assert _field(b, "threshold") == " ".join("%.17g" % v for v in t["threshold"])
        assert _field(b, "leaf_weight") == " ".join("%.17g" % v for v in t["leaf_weight"])
        assert _field(b, "split_gain") == " ".join("%g" % float(v) for v in t["split_gain"])
        assert _field(b, "internal_value") == " ".join("%g" % v for v in iv)
        assert _field(b, "internal_weight") == " ".join(["0"] * (t["num_leaves"] - 1))
        assert _field(b, "decision_type") == " ".join(["2"] * (t["num_leaves"] - 1))
        assert _field(b, "left_child") == " ".join(str(v) for v in t["left_child"])
    # split-count importances over splits with gain > 0, count-descending, stable
    counts = np.zeros(n_feat, np.int64)
    for t in trees:
        np.add.at(counts, t["split_feature"][t["split_gain"] > 0], 1)
    order = sorted([f for f in range(n_feat) if counts[f] > 0], key=lambda f: -counts[f])
    assert tail == "\nfeature_importances:\n" + "".join(f"Column_{f}={counts[f]}\n" for f in order)
    # the written text reads back to the same trees
    again = Model(text)
    assert again.to_text() == text
    ref = P.parse_model(text)
    X = rng.normal(size=(257, n_feat)).astype(np.float32) * 3
    raw = P.predict(ref, X, kind="raw")
    leaf = P.predict(ref, X, kind="leaf")
    exp = np.zeros(len(X))
    for k, t in enumerate(ref["trees"]):
        exp = exp + t["leaf_value"][leaf[:, k]]
    assert np.array_equal(raw[:, 0], exp)


def test_writer_constant_tree_and_names():
    m = Model.create(num_class=1, max_feature_idx=1, objective="regression",
                     feature_names="a b", feature_infos="[0:5] [0:2]")
    m.add_tree({"num_leaves": 1, "leaf_value": np.array([0.0]),
                "leaf_count": np.array([12], np.int32)}, shrinkage=1.0, bias=11.0)
    text = m.to_text()
    assert "\nfeature_names=a b\nfeature_infos=[0:5] [0:2]\n" in text
    assert ("Tree=0\nnum_leaves=1\nnum_cat=0\nsplit_feature=\nsplit_gain=\nthreshold=\n"
            "decision_type=\nleft_child=\nright_child=\nleaf_value=11\nleaf_weight=\n"
            "leaf_count=12\ninternal_value=\ninternal_weight=\ninternal_count=\nis_linear=0\n"
            "shrinkage=1\n\n\n") in text
    assert text.endswith("end of trees\n\nfeature_importances:\n")
    assert Model(text).to_text() == text


def test_writer_bias_rounds_to_zero():
    """Tree::add_bias applies MaybeRoundToZero (|v| <= 1e-35f -> 0) to every value."""
    m = Model.create(num_class=1, max_feature_idx=0, objective="regression")
    t = {"num_leaves": 2, "split_feature": np.array([0], np.int32), "threshold": np.array([0.5]),
         "split_gain": np.array([1.0], np.float32), "decision_type": np.array([2], np.int8),
         "left_child": np.array([-1], np.int32), "right_child": np.array([-2], np.int32),
         "internal_value": np.array([-0.25]), "internal_count": np.array([2], np.int32),
         "leaf_value": np.array([-0.25, 0.75]), "leaf_weight": np.array([1.0, 1.0]),
         "leaf_count": np.array([1, 1], np.int32)}
    m.add_tree(t, bias=0.25)
    b = m.to_text()
    assert "\nleaf_value=0 1\n" in b and "\ninternal_value=0\n" in b


@pytest.mark.parametrize("edit,needle", [
    (lambda t: t.update(right_child=np.array([5], np.int32)), "out of range"),
    (lambda t: t.update(split_feature=np.array([3], np.int32)), "split_feature"),
    (lambda t: t.update(num_leaves=0), "num_leaves"),
])
def test_add_tree_rejects_malformed(edit, needle):
    m = Model.create(num_class=1, max_feature_idx=0, objective="regression")
    t = {"num_leaves": 2, "split_feature": np.array([0], np.int32), "threshold": np.array([0.5]),
         "decision_type": np.array([2], np.int8), "left_child": np.array([-1], np.int32),
         "right_child": np.array([-2], np.int32), "leaf_value": np.array([1.0, 2.0])}
    edit(t)
    with pytest.raises(HipError) as e:
        m.add_tree(t)
    assert needle in str(e.value)
    assert m.num_trees == 0


def test_create_rejects_unsupported_objective():
    with pytest.raises(HipError) as e:
        Model.create(num_class=1, max_feature_idx=0, objective="lambdarank")
    assert "not supported" in str(e.value)


def test_oracle_average_output_divides_transformed_only():
    """RF (average_output): transformed = raw / iterations for an identity objective
    (predict.rs:338-349); raw is the plain sum."""
    text = open(os.path.join(HERE, "golden", "model_text", "rf_single_bag.txt")).read()
    m = P.parse_model(text)
    assert m["average_output"]
    X = np.random.default_rng(2).normal(size=(64, m["max_feature_idx"] + 1)).astype(np.float32)
    raw = P.predict(m, X, kind="raw")
    n = len(m["trees"]) // m["num_tree_per_iteration"]
    assert np.array_equal(P.predict(m, X, kind="transformed"), raw / float(n))


def test_oracle_transformed_needs_objective():
    text = open(os.path.join(HERE, "golden", "model_text", "custom_no_objective.txt")).read()
    m = P.parse_model(text)
    X = np.zeros((2, m["max_feature_idx"] + 1), np.float32)
    P.predict(m, X, kind="raw")
    with pytest.raises(ValueError):
        P.predict(m, X, kind="transformed")
