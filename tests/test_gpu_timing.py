"""The timing pass (lgbm_hip_set_timing) launches every kernel of an iteration on its
own with a start/stop event pair bound to it, behind a bounded device-side hold, and
without the per-tree graphs.  Its results must equal the graph-replayed iterations bit
for bit, and every timed family must be counted.
"""
import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend
from lightgbm_rs_amd.synth import config1_like, config3_binned
from oracle import oracle

pytestmark = pytest.mark.gpu
K_EPS = 1e-15


def say(*a):
    print(*a, flush=True)


def bits(a):
    return np.ascontiguousarray(a, np.float64).view(np.uint64)


def _same(ta, tb, tag):
    assert ta["num_leaves"] == tb["num_leaves"], tag
    for k in ta:
        if k == "num_leaves":
            continue
        a, b = np.ascontiguousarray(ta[k]), np.ascontiguousarray(tb[k])
        assert a.shape == b.shape and a.tobytes() == b.tobytes(), (tag, k)


def _binary_run(bins, meta, ub, y, init, timing, iters):
    cfg = GainConfig.make(min_data_in_leaf=20)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, ub)
        be.set_labels(y, init)
        be.set_timing(timing)
        trees = [be.train_iter_binary(i, cfg, 255, -1, 0.1, 4, True) for i in range(iters)]
        tm = be.timing() if timing else None
        return trees, be.scores(), tm
    finally:
        be.close()


def test_timed_binary_iterations_equal_graph_replay():
    n, iters = 400_000, 3
    bins, meta, ub, y = config1_like(n, seed=61)
    init = oracle.boost_from_score(y)
    say(f"timed binary iterations n={n}")
    plain, s_plain, _ = _binary_run(bins, meta, ub, y, init, False, iters)
    timed, s_timed, tm = _binary_run(bins, meta, ub, y, init, True, iters)
    for i, (a, b) in enumerate(zip(plain, timed)):
        _same(a, b, ("binary", i))
    assert np.array_equal(bits(s_plain), bits(s_timed))
    # every family of the iteration was timed
    for k in ("hist_ms", "partition_ms", "scan_ms", "quant_ms", "objective_ms"):
        assert tm[k] > 0.0, k
    assert tm["trees"] == iters
    assert tm["partition_launches"] >= tm["rounds"] > 0


def test_timed_multiclass_iteration_equals_graph_replay():
    n, K, nl = 60_000, 10, 31
    bins, meta, vals, y, _, _, _ = config3_binned(n, seed=0x5EED0061)
    prior = np.bincount(y.astype(np.int64), minlength=K) / n
    init = np.log(np.maximum(prior, K_EPS))
    applied = np.where(np.abs(init) > K_EPS, init, 0.0)
    cfg = GainConfig.make(min_data_in_leaf=20)
    say(f"timed multiclass iteration n={n} K={K}")
    out = []
    for timing in (False, True):
        be = HipBackend(0)
        try:
            be.upload_resident_bins(bins, meta, vals)
            be.set_labels_multiclass(y, K, applied)
            be.set_timing(timing)
            trees = be.train_iter_multiclass(0, cfg, nl, -1, 0.1, 4, True, [1] * K)
            out.append((trees, be.scores()))
        finally:
            be.close()
    (ta, sa), (tb, sb) = out
    assert len(ta) == len(tb) == K
    for k, (a, b) in enumerate(zip(ta, tb)):
        _same(a, b, ("multiclass", k))
    assert np.array_equal(bits(sa), bits(sb))
