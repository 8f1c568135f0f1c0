"""Binning on the host (no GPU): the library's BinMapper construction and ValueToBin
against the reference's binning goldens (bin_upper_bound_ bit-exact, mapper fields
and per-row bins exact), and the oracle's vectorised ValueToBin against the same
vectors (it checks the device kernel in tests/test_gpu_binning.py)."""
import numpy as np
import pytest

from tests import binning_fixtures as BF
from lightgbm_rs_amd import BinMapper, HipError, sample_indices
from oracle import binning as OB

NUMERIC = BF.cases("numeric_binning")
MISSING = BF.cases("missing_edge_cases")
CATEG = BF.cases("categorical_folding")
EXAMPLES = BF.datasets("example_dataset_binning")
INGEST = BF.datasets("default_config_ingest")
FIELDS = ("num_bin", "missing_type", "default_bin", "most_freq_bin", "is_trivial")


def _check_fields(m, exp, tag):
    for k in FIELDS:
        if k in exp:
            assert int(getattr(m, k)) == int(exp[k]), (tag, k, getattr(m, k), exp[k])
    if "bin_type" in exp:
        assert m.bin_type == int(exp["bin_type"]), tag
    if "upper" in exp:
        assert np.array_equal(m.upper_bounds.view(np.uint64), BF.bits_to_f64(exp["upper"]).view(np.uint64)), tag


def _oracle_bins(m, values):
    if m.bin_type == 1:
        return OB.value_to_bin_categorical(values, m.categories)
    return OB.value_to_bin_numeric(values, m.upper_bounds, m.missing_type)


def test_fixture_counts():
    assert (len(NUMERIC), len(MISSING), len(CATEG), len(EXAMPLES), len(INGEST)) == (45, 8, 6, 2, 1)


@pytest.mark.parametrize("case", NUMERIC, ids=lambda c: c["params"]["name"])
def test_find_bin_from_column_numeric_goldens(case):
    """numeric_assignment.rs:19-70: find_bin_from_column(column, max_bin,
    min_data_in_bin, min_split_data, pre_filter, use_missing, zero_as_missing,
    sample_cnt, seed)."""
    p = case["params"]
    m = BinMapper.from_column(
        case["values"], max_bin=int(p["max_bin"]), min_data_in_bin=int(p["min_data_in_bin"]),
        min_data_in_leaf=int(p["min_split_data"]), pre_filter=int(p["pre_filter"]),
        use_missing=int(p["use_missing"]), zero_as_missing=int(p["zero_as_missing"]),
        bin_construct_sample_cnt=int(p["sample_cnt"]), data_random_seed=int(p["seed"]))
    _check_fields(m, case["mapper"], p["name"])
    assert np.array_equal(m.value_to_bin(case["values"]), case["assign"])
    assert np.array_equal(_oracle_bins(m, case["values"]), case["assign"])


@pytest.mark.parametrize("case", MISSING, ids=lambda c: c["params"]["name"])
def test_missing_edge_cases_goldens(case):
    """missing_edge_cases.rs:150-170: find_bin_numeric over the whole column,
    min_data_in_bin 1, min_split_data 1, no pre-filter."""
    p = case["params"]
    v = case["values"]
    m = BinMapper.from_sample(v, len(v), min_split_data=1, max_bin=int(p["max_bin"]),
                              min_data_in_bin=1, pre_filter=False,
                              use_missing=int(p["use_missing"]),
                              zero_as_missing=int(p["zero_as_missing"]))
    _check_fields(m, case["mapper"], p["name"])
    assert np.array_equal(m.value_to_bin(v), case["assign"])
    assert np.array_equal(_oracle_bins(m, v), case["assign"])


@pytest.mark.parametrize("case", CATEG, ids=lambda c: c["params"]["name"])
def test_categorical_folding_goldens(case):
    """categorical_folding.rs:205-260: find_bin_categorical over the whole column."""
    p = case["params"]
    v = case["values"]
    m = BinMapper.from_sample(v, len(v), categorical=True,
                              min_split_data=int(p["min_split_data"]), max_bin=int(p["max_bin"]),
                              min_data_in_bin=int(p["min_data_in_bin"]),
                              pre_filter=int(p["pre_filter"]), use_missing=int(p["use_missing"]),
                              zero_as_missing=int(p["zero_as_missing"]))
    _check_fields(m, case["mapper"], p["name"])
    assert np.array_equal(m.categories, case["b2c"])
    assert {int(c): b for b, c in enumerate(m.categories)} == case["c2b"]
    assert np.array_equal(m.value_to_bin(v), case["assign"])
    assert np.array_equal(_oracle_bins(m, v), case["assign"])


@pytest.mark.parametrize("ds", EXAMPLES, ids=lambda d: d["params"]["name"])
def test_example_dataset_goldens(ds):
    """example_dataset_parity.rs:183-240: find_bin_from_column(column, 255, 3, 20,
    no pre-filter, use_missing, sample 100000 rows, the dataset's seed)."""
    X = BF.examples()[ds["params"]["name"].split(".")[0]]
    assert X.shape == (int(ds["params"]["num_rows"]), int(ds["params"]["num_features"]))
    for f in range(X.shape[1]):
        m = BinMapper.from_column(X[:, f], max_bin=255, min_data_in_bin=3, min_data_in_leaf=20,
                                  pre_filter=False, bin_construct_sample_cnt=100000,
                                  data_random_seed=int(ds["params"]["seed"]))
        _check_fields(m, ds["features"][f], f)
        assert np.array_equal(m.value_to_bin(X[:, f]), ds["assign"][f]), f
        assert np.array_equal(_oracle_bins(m, X[:, f]), ds["assign"][f]), f


def test_default_config_ingest_golden():
    """default_config_ingest_parity.rs: feature_pre_filter on, 50 of 200 rows sampled,
    the pre-filter threshold scaled to min_data_in_leaf * 50 / 200."""
    ds = INGEST[0]
    p = ds["params"]
    X = ds["matrix"]
    for f in range(X.shape[1]):
        exp = ds["features"][f]
        m = BinMapper.from_column(X[:, f], max_bin=int(p["max_bin"]),
                                  min_data_in_bin=int(p["min_data_in_bin"]),
                                  min_data_in_leaf=int(p["min_data_in_leaf"]), pre_filter=True,
                                  bin_construct_sample_cnt=int(p["bin_construct_sample_cnt"]),
                                  data_random_seed=int(p["seed"]))
        _check_fields(m, exp, f)
    assert any(int(e["is_trivial"]) for e in ds["features"].values())


def test_sample_indices_properties():
    for n, k, seed in [(1000, 64, 3), (1000, 900, 4), (50, 50, 5), (200, 50, 185716609), (7, 100, 1)]:
        idx = sample_indices(n, k, seed)
        assert len(idx) == min(n, k)
        assert np.all(np.diff(idx) > 0) and idx[0] >= 0 and idx[-1] < n
    assert np.array_equal(sample_indices(9, 9, 1), np.arange(9))
    assert len(sample_indices(10, 0, 1)) == 0


def test_value_to_bin_vs_oracle_random():
    """Library ValueToBin vs the oracle on values at, around and between the bounds,
    signed zeros, NaN and infinities."""
    rng = np.random.default_rng(12)
    base = np.concatenate([rng.normal(size=5000), np.zeros(500), rng.integers(-5, 5, 1000) * 1.0])
    base[rng.random(len(base)) < 0.05] = np.nan
    for kw in [dict(), dict(zero_as_missing=True), dict(use_missing=False), dict(max_bin=16)]:
        m = BinMapper.from_column(base, **kw)
        ub = m.upper_bounds[np.isfinite(m.upper_bounds)]
        probe = np.concatenate([base, ub, np.nextafter(ub, np.inf), np.nextafter(ub, -np.inf),
                                [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-35, -1e-35, 1e300]])
        assert np.array_equal(m.value_to_bin(probe), _oracle_bins(m, probe)), kw


def test_from_column_rejects_bad_params():
    with pytest.raises(HipError):
        BinMapper.from_column(np.zeros(10), max_bin=1)
    with pytest.raises(TypeError):
        BinMapper.from_column(np.zeros(10), maxbin=10)


def test_from_sampled_column_equals_from_column():
    """Gathering the sample rows outside the library gives the same mapper."""
    rng = np.random.default_rng(21)
    col = rng.normal(size=30000)
    col[rng.random(30000) < 0.1] = 0.0
    col[rng.random(30000) < 0.02] = np.nan
    for kw in [dict(bin_construct_sample_cnt=5000, data_random_seed=9, max_bin=63),
               dict(bin_construct_sample_cnt=50000, max_bin=255),
               dict(bin_construct_sample_cnt=1000, pre_filter=True, min_data_in_leaf=500)]:
        a = BinMapper.from_column(col, **kw)
        idx = sample_indices(len(col), kw["bin_construct_sample_cnt"], kw.get("data_random_seed", 1))
        b = BinMapper.from_sampled_column(col[idx], len(col), **kw)
        assert np.array_equal(a.upper_bounds.view(np.uint64), b.upper_bounds.view(np.uint64))
        for k in ("num_bin", "missing_type", "default_bin", "most_freq_bin", "is_trivial"):
            assert getattr(a, k) == getattr(b, k), k
