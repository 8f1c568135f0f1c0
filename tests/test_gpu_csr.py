"""Device prediction from CSR rows (`lgbm_hip_predict_csr`; predict_raw_csr_range /
predict_leaf_index_csr / predict_contrib_csr, crates/lgbm-model/src/predict.rs:132-160,
485-500, 699-722, with scatter_csr_row / validate_indptr_pair, predict.rs:772-870).

Bars: for every kind, bits equal to the dense predictor on the same rows made dense
by the reference's rule (zeros elsewhere, a repeated column keeps its last value,
columns past max_feature_idx dropped), with empty rows, NaN values and repeated
columns in the input; malformed indptr pairs and out-of-range columns refused with
the reference's two error kinds."""
import os

import numpy as np
import pytest

from lightgbm_rs_amd import HipBackend, HipError, Model
from oracle import predict as P

pytestmark = pytest.mark.gpu
MT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_text")


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


def random_csr(rng, rows, num_cols, per_row):
    counts = rng.integers(0, per_row + 1, size=rows)
    counts[::7] = 0  # empty rows
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    nnz = int(indptr[-1])
    indices = rng.integers(0, num_cols, size=nnz).astype(np.int32)  # repeats allowed
    values = rng.normal(scale=2.0, size=nnz).astype(np.float32)
    values[rng.random(nnz) < 0.05] = np.nan
    return indptr, indices, values


def densify(indptr, indices, values, width):
    X = np.zeros((len(indptr) - 1, width), np.float32)
    for r in range(len(indptr) - 1):
        for k in range(indptr[r], indptr[r + 1]):
            if indices[k] < width:
                X[r, indices[k]] = values[k]
    return X


@pytest.mark.parametrize("name", ["binary_spine", "multiclass_spine", "cat_manyvsmany",
                                  "na_missing"])
def test_csr_predict_equals_dense(be, name):
    print("csr", name, flush=True)
    text = open(os.path.join(MT, name + ".txt")).read()
    m = Model(text)
    width = P.parse_model(text)["max_feature_idx"] + 1
    rng = np.random.default_rng(21)
    num_cols = width + 3
    indptr, indices, values = random_csr(rng, 5003, num_cols, 2 * width)
    X = densify(indptr, indices, values, width)
    for kind in ("raw", "leaf", "contrib"):
        got = be.predict_csr(m, indptr, indices, values, num_cols, kind)
        ref = be.predict(m, X, kind)
        assert got.dtype == ref.dtype and np.array_equal(got.view(np.uint8), ref.view(np.uint8)), kind
    got = be.predict_csr(m, indptr, indices, values, num_cols, "raw", start_iteration=1,
                         num_iteration=1)
    assert np.array_equal(got, be.predict(m, X, "raw", start_iteration=1, num_iteration=1))


def test_csr_errors(be):
    print("csr errors", flush=True)
    m = Model(open(os.path.join(MT, "binary_spine.txt")).read())
    ind = np.array([0, 1, 0], np.int32)
    val = np.ones(3, np.float32)
    for bad in ([0, 2, 1, 3], [0, 1, 4, 4], [-1, 1, 2, 3]):
        with pytest.raises(HipError, match="malformed indptr"):
            be.predict_csr(m, np.array(bad, np.int64), ind, val, 2)
    with pytest.raises(HipError, match="column index out of range"):
        be.predict_csr(m, np.array([0, 1, 2, 3], np.int64), np.array([0, 2, 1], np.int32), val, 2)
    with pytest.raises(HipError, match="column index out of range"):
        be.predict_csr(m, np.array([0, 1, 2, 3], np.int64), np.array([0, -1, 1], np.int32), val, 2)
    with pytest.raises(HipError, match="columns"):
        be.predict_csr(m, np.array([0, 1, 2, 3], np.int64), ind, val, 1)
    # a valid call after the refusals
    got = be.predict_csr(m, np.array([0, 1, 2, 3], np.int64), ind, val, 2)
    assert np.array_equal(got, be.predict(m, densify([0, 1, 2, 3], ind, val, 2), "raw"))


def to_csc(indptr, indices, values, num_cols):
    """The same entries column by column, each column's entries in row order (so a
    repeated (row, column) keeps the value the CSR rule keeps: the last)."""
    rows = np.repeat(np.arange(len(indptr) - 1), np.diff(indptr))
    order = np.lexsort((np.arange(len(indices)), rows, indices))
    cptr = np.concatenate([[0], np.cumsum(np.bincount(indices, minlength=num_cols))])
    return cptr.astype(np.int64), rows[order].astype(np.int32), values[order]


@pytest.mark.parametrize("name", ["binary_spine", "multiclass_spine", "cat_manyvsmany"])
def test_csc_predict_equals_dense(be, name):
    print("csc", name, flush=True)
    text = open(os.path.join(MT, name + ".txt")).read()
    m = Model(text)
    width = P.parse_model(text)["max_feature_idx"] + 1
    rng = np.random.default_rng(22)
    num_cols = width + 2
    indptr, indices, values = random_csr(rng, 4001, num_cols, 2 * width)
    X = densify(indptr, indices, values, width)
    cptr, rows, vals = to_csc(indptr, indices, values, num_cols)
    for kind in ("raw", "leaf", "contrib"):
        got = be.predict_csc(m, cptr, rows, vals, len(indptr) - 1, kind)
        ref = be.predict(m, X, kind)
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), kind


def test_csc_errors(be):
    print("csc errors", flush=True)
    m = Model(open(os.path.join(MT, "binary_spine.txt")).read())
    rows = np.array([0, 1, 2], np.int32)
    val = np.ones(3, np.float32)
    with pytest.raises(HipError, match="malformed indptr"):
        be.predict_csc(m, np.array([0, 2, 1], np.int64), rows, val, 3)
    with pytest.raises(HipError, match="row index out of range"):
        be.predict_csc(m, np.array([0, 2, 3], np.int64), rows, val, 2)
    got = be.predict_csc(m, np.array([0, 2, 3], np.int64), rows, val, 3)
    X = np.array([[1, 0], [1, 0], [0, 1]], np.float32)
    assert np.array_equal(got, be.predict(m, X, "raw"))


def test_csc_repeated_rows_keep_the_last_entry(be):
    """Entries of a column are placed in parallel; a row repeated anywhere in its
    column (not only next to itself) keeps the column's last value."""
    print("csc repeated rows", flush=True)
    m = Model(open(os.path.join(MT, "binary_spine.txt")).read())
    cptr = np.array([0, 3, 5], np.int64)
    rows = np.array([2, 0, 2, 1, 1], np.int32)
    vals = np.array([5, 1, 7, 3, 9], np.float32)
    got = be.predict_csc(m, cptr, rows, vals, 3)
    X = np.array([[1, 0], [0, 9], [7, 0]], np.float32)
    assert np.array_equal(got, be.predict(m, X, "raw"))


def test_csc_tall_columns_equal_dense(be):
    """A tall input of few columns (the shape a per-column pass serialises): random
    entries with repeated rows, against the dense prediction of the same values."""
    print("csc tall", flush=True)
    m = Model(open(os.path.join(MT, "binary_spine.txt")).read())
    rng = np.random.default_rng(31)
    n, cols = 300_000, 3
    cptr = [0]
    rows_l, vals_l = [], []
    X = np.zeros((n, 2), np.float32)
    for c in range(cols):
        k = int(rng.integers(n // 2, n))
        r = rng.integers(0, n, size=k).astype(np.int32)  # repeats in any order
        v = rng.standard_normal(k).astype(np.float32)
        if c < 2:
            X[r, c] = v  # numpy keeps the last assignment of a repeated index
        rows_l.append(r)
        vals_l.append(v)
        cptr.append(cptr[-1] + k)
    got = be.predict_csc(m, np.array(cptr, np.int64), np.concatenate(rows_l),
                         np.concatenate(vals_l), n)
    assert np.array_equal(got, be.predict(m, X, "raw"))
