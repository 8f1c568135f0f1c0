"""HIP path vs the CPU oracle (and the reference's golden vectors), on a real MI355X.

Bar: bit-exact for every integer / index result and for every f64 produced in the
quantized (integer-exact) mode; the oracle is tests' checker only.
"""
import json
import os
import struct
import sys

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend
from lightgbm_rs_amd._abi import BatchedFeature
from oracle import oracle
from tests.datagen import binary_gh, config1_like, make_binned

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint64 if a.dtype == np.float64 else np.uint32)


def b64(x):
    return struct.unpack("<Q", struct.pack("<d", float(x)))[0]


def f64(bitlist):
    return np.array(bitlist, dtype=np.uint64).view(np.float64)


def slot_layout(meta):
    offs, acc = [], 0
    for m in meta:
        offs.append(acc)
        acc += 2 * m.num_bin
    return offs, acc


# ---------------------------------------------------------------------------
# quantizer
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,stochastic,seed", [(1000, False, 0), (1000, True, 3),
                                               (300_001, True, 0x51702010),
                                               (2_500_000, True, (7 << 20) ^ 0x51702010)])
def test_quantize_matches_oracle(be, n, stochastic, seed):
    say(f"quantize n={n} stochastic={stochastic} seed={seed}")
    bins, meta, ub = make_binned(n, 3, seed=1)
    g, h, _ = binary_gh(n, seed=2)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)
    scales, dg, dh = be.discretize_dequantize_in_place(4, stochastic, seed, want_values=True)
    og, oh, disc, oscales = oracle.quantize(g, h, bins=4, stochastic=stochastic, seed=seed)
    assert np.array_equal(bits(scales), bits(oscales))
    assert np.array_equal(be.discretized(), disc)
    assert np.array_equal(bits(dg), bits(og))
    assert np.array_equal(bits(dh), bits(oh))


def test_quantize_constant_hessian(be):
    n = 5000
    bins, meta, ub = make_binned(n, 2, seed=4)
    g = np.random.default_rng(5).normal(size=n).astype(np.float32)
    h = np.ones(n, np.float32)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)
    scales, dg, dh = be.discretize_dequantize_in_place(4, True, 11, want_values=True)
    og, oh, disc, osc = oracle.quantize(g, h, bins=4, stochastic=True, seed=11)
    assert np.array_equal(be.discretized(), disc)
    assert np.array_equal(bits(scales), bits(osc))


# ---------------------------------------------------------------------------
# ConstructHistogram
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,F,subset", [(20_000, 7, False), (20_000, 7, True),
                                        (1_000_003, 28, False), (1_000_003, 28, True)])
def test_int_histogram_matches_oracle(be, n, F, subset):
    say(f"int histogram n={n} F={F} subset={subset}")
    bins, meta, ub = make_binned(n, F, seed=n + F)
    g, h, _ = binary_gh(n, seed=3)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)
    be.discretize_dequantize_in_place(4, True, 99)
    disc = be.discretized()
    rows = None
    if subset:
        rows = np.sort(np.random.default_rng(7).choice(n, size=n // 3, replace=False)).astype(np.uint32)
    got = be.construct_int_histogram(rows)
    offs, total = slot_layout(meta)
    r = np.arange(n, dtype=np.uint32) if rows is None else rows
    for f, m in enumerate(meta):
        exp = oracle.int_histogram(bins[f].astype(np.uint32), disc, r, m.num_bin)
        assert np.array_equal(got[offs[f]:offs[f] + 2 * m.num_bin], exp), f"feature {f}"


@pytest.mark.parametrize("n,F", [(30_000, 9), (400_000, 28)])
def test_leaf_histogram_bit_exact_vs_f64_fold(be, n, F):
    """Integer build + exact f64 conversion + FixHistogram + compaction equals the
    reference's ascending-row f64 fold of the dequantized values (build_leaf_histogram_into)."""
    say(f"leaf histogram n={n} F={F}")
    bins, meta, ub = make_binned(n, F, seed=F)
    g, h, _ = binary_gh(n, seed=5)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)
    _, dg, dh = be.discretize_dequantize_in_place(4, True, 1234, want_values=True)
    rows = np.sort(np.random.default_rng(1).choice(n, size=n // 2, replace=False)).astype(np.uint32)
    # leaf sums with kEpsilon-style provenance (not exactly the fold) to exercise the fix
    sg = float(np.sum(dg[rows].astype(np.float64))) + 1e-15
    sh = float(np.sum(dh[rows].astype(np.float64))) + 2e-15
    got = be.build_resident_leaf(rows, sg, sh)
    offs, total = slot_layout(meta)
    for f, m in enumerate(meta):
        hist = oracle.construct_histogram(bins[f][rows], dg[rows], dh[rows], m.num_bin)
        hist = oracle.fix_histogram(hist, m.num_bin, m.most_freq_bin, sg, sh)
        hist = oracle.compact_histogram(hist, m.num_bin, m.offset)
        assert np.array_equal(bits(got[offs[f]:offs[f] + 2 * m.num_bin]), bits(hist)), f"feature {f}"


# ---------------------------------------------------------------------------
# FindBestThreshold
# ---------------------------------------------------------------------------
def _golden_cfg(c):
    return GainConfig.make(min_data_in_leaf=c["min_data_in_leaf"],
                           min_sum_hessian_in_leaf=f64([c["min_sum_hessian_in_leaf_bits"]])[0],
                           lambda_l1=f64([c["lambda_l1_bits"]])[0],
                           lambda_l2=f64([c["lambda_l2_bits"]])[0],
                           min_gain_to_split=f64([c["min_gain_to_split_bits"]])[0])


def test_find_best_splits_golden(be):
    """kernels/split.txt winners (kernel_parity.rs:512), bit-exact on the device scan."""
    cases = json.load(open(os.path.join(GOLD, "split_scan.json")))
    for c in cases:
        bf = BatchedFeature(0, c["num_bin"], c["offset"], c["default_bin"], 0,
                            c["skip_default_bin"], c["na_as_missing"], 1, 0)
        [si] = be.find_best_splits_batched(f64(c["hist_bits"]), [bf], _golden_cfg(c),
                                           f64([c["sum_gradient_bits"]])[0],
                                           f64([c["sum_hessian_bits"]])[0], c["num_data"])
        w = c["win"]
        assert (si.gain == -np.inf) == (not w["is_splittable"]), c["name"]
        if w["is_splittable"]:
            for k in ["gain", "left_sum_gradient", "left_sum_hessian", "right_sum_gradient",
                      "right_sum_hessian", "left_output", "right_output"]:
                assert b64(getattr(si, k)) == w[k + "_bits"], (c["name"], k)
            assert (si.threshold, si.left_count, si.right_count, si.default_left) == (
                w["threshold"], w["left_count"], w["right_count"], w["default_left"]), c["name"]


def _random_scan_case(rng, nb):
    g = rng.normal(0, 1, nb) * (rng.random(nb) < 0.9)
    h = rng.random(nb) * 3 * (rng.random(nb) < 0.9)
    hist = np.empty(2 * nb)
    hist[0::2], hist[1::2] = g, h
    return hist


@pytest.mark.parametrize("seed", range(6))
def test_find_best_splits_random_vs_oracle(be, seed):
    rng = np.random.default_rng(seed)
    feats, hists = [], []
    off = 0
    for j in range(24):
        nb = int(rng.choice([2, 3, 5, 17, 63, 64, 65, 130, 256]))
        mt = int(rng.integers(0, 3)) if nb > 2 else 0
        offset = int(rng.integers(0, 2))
        defb = int(rng.integers(0, nb + 1))
        hist = _random_scan_case(rng, nb)
        feats.append(BatchedFeature(off, nb, offset, defb, 0, int(nb > 2 and mt == 1),
                                    int(nb > 2 and mt == 2), int(nb > 2 and mt != 0), 0))
        hists.append(hist)
        off += 2 * nb
    allh = np.concatenate(hists)
    cfgs = [GainConfig.make(min_data_in_leaf=int(rng.integers(0, 30)),
                            min_sum_hessian_in_leaf=float(rng.choice([0.0, 1e-3, 0.5]))),
            GainConfig.make(min_data_in_leaf=3, lambda_l1=0.3, lambda_l2=1.5, min_gain_to_split=0.1),
            GainConfig.make(min_data_in_leaf=2, max_delta_step=0.7),
            GainConfig.make(min_data_in_leaf=2, path_smooth=2.0, lambda_l2=0.5)]
    for cfg in cfgs:
        cfg.parent_output = float(rng.normal())
        sg = float(rng.normal() * 5)
        sh = float(rng.random() * 40 + 1)
        n = int(rng.integers(50, 5000))
        got = be.find_best_splits_batched(allh, feats, cfg, sg, sh, n)
        for j, bf in enumerate(feats):
            exp = oracle.find_best_split(hists[j], cfg, bf.num_bin, bf.offset, bf.default_bin,
                                         bf.skip_default_bin, bf.na_as_missing, bf.run_forward,
                                         sg, sh, n)
            gd, ed = got[j].as_dict(), exp.as_dict()
            for k in ed:
                if isinstance(ed[k], float):
                    assert b64(gd[k]) == b64(ed[k]), (seed, j, k, gd[k], ed[k])
                else:
                    assert gd[k] == ed[k], (seed, j, k)


# ---------------------------------------------------------------------------
# subtract / partition
# ---------------------------------------------------------------------------
def test_subtract_golden(be):
    for c in json.load(open(os.path.join(GOLD, "subtract.json"))):
        got = be.subtract_histograms(f64(c["parent_bits"]), f64(c["child_bits"]))
        assert np.array_equal(bits(got), np.array(c["derived_bits"], dtype=np.uint64))


def test_partition_golden(be):
    for c in json.load(open(os.path.join(GOLD, "partition.json"))):
        if c["missing_type"] != 0:
            continue
        order, split = be.data_partition(c["bins"], c["num_bin"], c["min_bin"], c["max_bin"],
                                         c["threshold"], c["most_freq_bin"])
        assert order.tolist() == c["order"], c["name"]
        assert split == c["split_point"], c["name"]


@pytest.mark.parametrize("n", [1, 2047, 2048, 2049, 100_000, 1_234_567])
def test_partition_random_vs_oracle(be, n):
    say(f"partition n={n}")
    rng = np.random.default_rng(n)
    nb = 64
    bins = rng.integers(0, nb, n).astype(np.uint32)
    for (mn, mx, thr, mfb, na, dl) in [(0, 63, 20, 0, 0, 0), (1, 62, 40, 5, 1, 1),
                                       (0, 63, 62, 63, 1, 0), (3, 10, 5, 0, 0, 0)]:
        got, gl = be.data_partition(bins, nb, mn, mx, thr, mfb, na, dl)
        exp, el = oracle.data_partition(bins, nb, mn, mx, thr, mfb, na, dl)
        assert gl == el
        assert np.array_equal(got, exp)


def test_partition_errors(be):
    from lightgbm_rs_amd import HipError
    with pytest.raises(HipError) as e:
        be.data_partition([0, 9], 8, 0, 7, 3, 0)
    assert e.value.code == -2
    with pytest.raises(HipError) as e:
        be.data_partition([0, 1], 8, 0, 7, 8, 0)
    assert e.value.code == -4


# ---------------------------------------------------------------------------
# whole tree (coarse seam) vs the oracle learner
# ---------------------------------------------------------------------------
def _compare_trees(t, o, tag):
    assert t["num_leaves"] == o["num_leaves"], tag
    for k in o:
        if k == "num_leaves":
            continue
        a, b = np.asarray(t[k]), np.asarray(o[k])
        if a.dtype.kind == "f":
            assert np.array_equal(bits(a), bits(b)), (tag, k)
        else:
            assert np.array_equal(a, b), (tag, k)


@pytest.mark.parametrize("n,F,nl,md,seed", [
    (500, 3, 8, -1, 1),
    (20_000, 9, 31, -1, 2),
    (20_000, 9, 63, 4, 3),
    (200_000, 28, 255, -1, 4),
])
def test_grow_tree_matches_oracle(be, n, F, nl, md, seed):
    say(f"grow_tree n={n} F={F} num_leaves={nl} max_depth={md}")
    bins, meta, ub = make_binned(n, F, seed=seed)
    g, h, _ = binary_gh(n, seed=seed)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)
    _, dg, dh = be.discretize_dequantize_in_place(4, True, seed * 77, want_values=True)
    og, oh, _, _ = oracle.quantize(g, h, bins=4, stochastic=True, seed=seed * 77)
    assert np.array_equal(bits(dg), bits(og))
    cfg = GainConfig.make(min_data_in_leaf=20)
    t, lay = be.grow_tree_on_device_with_cfg(cfg, nl, md)
    o, olay = oracle.train_tree(bins, meta, ub, og, oh, cfg, nl, md)
    _compare_trees(t, o, (n, F, nl))
    assert np.array_equal(lay["leaf_begin"], olay["leaf_begin"])
    assert np.array_equal(lay["leaf_count"], olay["leaf_count"])
    assert np.array_equal(lay["indices"], olay["indices"])


def test_grow_tree_config1_shape(be):
    """Config-1 shaped (quantile-binned, 28 features, max_bin 63, 255 leaves) at 1M rows."""
    n = 1_000_000
    say(f"grow_tree config1-like n={n}")
    bins, meta, ub, y = config1_like(n)
    g, h, _ = binary_gh(n, seed=9)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)
    _, dg, dh = be.discretize_dequantize_in_place(4, True, 0x51702010, want_values=True)
    og, oh, _, _ = oracle.quantize(g, h, bins=4, stochastic=True, seed=0x51702010)
    cfg = GainConfig.make(min_data_in_leaf=20)
    t, lay = be.grow_tree_on_device_with_cfg(cfg, 255, -1)
    o, olay = oracle.train_tree(bins, meta, ub, og, oh, cfg, 255, -1)
    _compare_trees(t, o, "config1")
    assert np.array_equal(lay["indices"], olay["indices"])


def _mrz(v):
    z = float(np.float32(1e-35))
    return np.where((v >= -z) & (v <= z), 0.0, v)


def compare_boosted(trees, scores, otrees, oscores, init, tag):
    """Device iterations vs the oracle's boosting loop, every field bit-exact.  The
    oracle's first tree carries Tree::add_bias(init) (tree.rs:1161); the device
    returns the shrunk tree and keeps the bias in the scores."""
    assert len(trees) == len(otrees), tag
    for i, (t, o) in enumerate(zip(trees, otrees)):
        t = dict(t)
        if i == 0 and init != 0.0:
            t["leaf_value"] = _mrz(t["leaf_value"] + init)
            t["internal_value"] = _mrz(t["internal_value"] + init)
        _compare_trees(t, o, (tag, i))
    assert np.array_equal(bits(scores), bits(oscores)), tag


def test_train_binary_matches_oracle(be):
    """Five resident boosting iterations (objective -> quantize -> grow -> score):
    trees and training scores bit-exact."""
    n, iters, nl = 50_000, 5, 31
    bins, meta, ub, y = config1_like(n, seed=3)
    init = oracle.boost_from_score(y)
    be.upload_resident_bins(bins, meta, ub)
    be.set_labels(y, init)
    cfg = GainConfig.make(min_data_in_leaf=20)
    trees = [be.train_iter_binary(i, cfg, nl, -1, 0.1) for i in range(iters)]
    scores = be.scores()
    oscores, otrees = oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, iters, 0.1)
    compare_boosted(trees, scores, otrees, oscores, init, "train_binary")


def test_config1_full_size_chain_matches_oracle():
    """BASELINE configs[1] at its full size through the chain bench.py times: the raw
    10.5M x 28 table -> BinMapper on the 200000-row sample -> device binning
    (lgbm_hip_upload_raw) -> resident quantized boosting (4 bins, stochastic, 255
    leaves).  Two iterations against the oracle's boosting loop on the device's own
    bins: every tree field and every training score bit-exact
    (gbdt.rs:691-1160)."""
    from lightgbm_rs_amd import BinMapper, binary_boost_from_score, feature_meta, sample_indices
    from lightgbm_rs_amd.synth import config1_raw_host
    n, iters, nl = 10_500_000, 2, 255
    say(f"config1 full-size chain n={n} iterations={iters}")
    X, y = config1_raw_host(n)
    idx = sample_indices(n, 200000, 1)
    ms = [BinMapper.from_sampled_column(X[f, idx].astype(np.float64), n, max_bin=63)
          for f in range(28)]
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    assert any(m.most_freq_bin > 0 for m in meta) and any(m.most_freq_bin == 0 for m in meta)
    ub = np.concatenate([m.upper_bounds for m in ms])
    init = binary_boost_from_score(y)
    cfg = GainConfig.make(min_data_in_leaf=20, min_sum_hessian_in_leaf=1e-3)
    b = HipBackend(0)
    try:
        b.upload_raw(X, ms, col_major=True)
        b.set_labels(y, init)
        trees = [b.train_iter_binary(i, cfg, nl, -1, 0.1, 4, True) for i in range(iters)]
        scores = b.scores()
        bins = b.get_bins()
    finally:
        b.close()
    del X
    say("  device done, oracle ...")
    oscores, otrees = oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, iters, 0.1,
                                          boost_from_average=True, quantized=True, quant_bins=4,
                                          stochastic=True)
    assert trees[0]["num_leaves"] == nl
    compare_boosted(trees, scores, otrees, oscores, init, "config1 full size")


def test_graph_replays_match_eager():
    """The captured per-tree graph, replayed with fresh gradients between eager work and
    synchronizations, grows exactly the trees the per-launch path grows."""
    n = 100_000
    bins, meta, ub = make_binned(n, 11, seed=21)
    os.environ["LGBM_HIP_GRAPHS"] = "0"
    try:
        eager = HipBackend(0)
    finally:
        del os.environ["LGBM_HIP_GRAPHS"]
    graph = HipBackend(0)
    try:
        for be_ in (eager, graph):
            be_.upload_resident_bins(bins, meta, ub)
        cfg = GainConfig.make(min_data_in_leaf=20)
        for rep in range(4):
            g, h, _ = binary_gh(n, seed=100 + rep)
            outs = []
            for be_ in (eager, graph):
                be_.upload_resident_grad_hess(g, h)
                be_.discretize_dequantize_in_place(4, True, rep)
                outs.append(be_.grow_tree_on_device_with_cfg(cfg, 63, -1))
            _compare_trees(outs[1][0], outs[0][0], ("replay", rep))
            assert np.array_equal(outs[1][1]["indices"], outs[0][1]["indices"])
    finally:
        eager.close()
        graph.close()


@pytest.mark.parametrize("spec,rounds", [(1, 300), (3, 2), (16, 1), (16, 64)])
def test_speculative_rounds_match_oracle(spec, rounds):
    """Leaves split ahead of their turn (up to `spec` per round) and any number of
    captured rounds (too few ones are completed by eager rounds) grow the oracle's
    tree: commits follow the reference's ArgMax order regardless."""
    n, F, nl = 150_000, 13, 127
    say(f"speculative rounds spec={spec} rounds={rounds}")
    bins, meta, ub = make_binned(n, F, seed=31)
    g, h, _ = binary_gh(n, seed=31)
    os.environ["LGBM_HIP_SPEC"] = str(spec)
    os.environ["LGBM_HIP_ROUNDS"] = str(rounds)
    try:
        b = HipBackend(0)
    finally:
        del os.environ["LGBM_HIP_SPEC"]
        del os.environ["LGBM_HIP_ROUNDS"]
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.upload_resident_grad_hess(g, h)
        _, dg, dh = b.discretize_dequantize_in_place(4, True, 5, want_values=True)
        og, oh, _, _ = oracle.quantize(g, h, bins=4, stochastic=True, seed=5)
        cfg = GainConfig.make(min_data_in_leaf=20)
        b.set_timing(True)
        t, lay = b.grow_tree_on_device_with_cfg(cfg, nl, -1)
        tm = b.timing()
        say(f"  rounds {tm['rounds']:.0f}, jobs {tm['partition_jobs']:.0f}, leaves {t['num_leaves']}")
        o, olay = oracle.train_tree(bins, meta, ub, og, oh, cfg, nl, -1)
        _compare_trees(t, o, ("spec", spec, rounds))
        assert np.array_equal(lay["indices"], olay["indices"])
        assert tm["partition_jobs"] >= t["num_leaves"] - 1
        if spec == 1:
            assert tm["partition_jobs"] == t["num_leaves"] - 1
    finally:
        b.close()


@pytest.mark.parametrize("blocks", [1, 37, 1000])
def test_partition_grid_shapes_match_oracle(blocks):
    """Partition launches of any width grow the oracle's tree: one block (all tiles of
    the root job in one block, so its histogram is flushed mid-job into the same
    slot), an odd width (slots of narrow jobs, accumulators of wide ones), and more
    blocks than tiles (blocks without tiles inside a job's block span)."""
    n, nl = 600_000, 63
    say(f"partition grid blocks={blocks}")
    bins, meta, ub, _ = config1_like(n, seed=41)
    g, h, _ = binary_gh(n, seed=41)
    os.environ["LGBM_HIP_PART_BLOCKS"] = str(blocks)
    try:
        b = HipBackend(0)
    finally:
        del os.environ["LGBM_HIP_PART_BLOCKS"]
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.upload_resident_grad_hess(g, h)
        _, dg, dh = b.discretize_dequantize_in_place(4, True, 7, want_values=True)
        og, oh, _, _ = oracle.quantize(g, h, bins=4, stochastic=True, seed=7)
        cfg = GainConfig.make(min_data_in_leaf=20)
        t, lay = b.grow_tree_on_device_with_cfg(cfg, nl, -1)
        o, olay = oracle.train_tree(bins, meta, ub, og, oh, cfg, nl, -1)
        _compare_trees(t, o, ("grid", blocks))
        assert np.array_equal(lay["indices"], olay["indices"])
    finally:
        b.close()


def test_tied_leaf_gains_break_by_leaf_id(be):
    """Mirrored groups: rows of group B repeat the bins of group A except for a marker
    feature and carry negated gradients (deterministic rounding keeps q(-g) = -q(g));
    group C (marker bin 2) is unrelated, so every feature has a real gain at the root.
    Once the marker splits off A, B and C, gains depend on G^2, so every leaf of A's
    subtree has a twin in B's with a bit-identical gain and feature: the cross-leaf
    ArgMax must break those ties by the lower leaf id, as the reference's sequential
    strict-> scan does."""
    na, nc_, F = 30_000, 20_000, 8
    b0, meta0, ub0 = make_binned(na + nc_, F - 1, seed=41, missing_mix=False, mfb_mix=False)
    n = 2 * na + nc_
    bins = np.zeros((F, n), dtype=np.uint8)
    bins[0, na:2 * na] = 1
    bins[0, 2 * na:] = 2
    bins[1:, :na] = b0[:, :na]
    bins[1:, na:2 * na] = b0[:, :na]
    bins[1:, 2 * na:] = b0[:, na:]
    from lightgbm_rs_amd import feature_meta
    meta = [feature_meta(3, real_index=0)]
    for i, m in enumerate(meta0):
        m.real_feature_index = i + 1
        meta.append(m)
    ub = np.concatenate([np.array([0.5, 1.5, 2.5]), ub0])
    ga, ha, _ = binary_gh(na, seed=41)
    # one sign per mirrored group (the marker splits first), and a signal on features
    # 1 and 4 so that the twin subtrees keep splitting
    ga = (np.abs(ga) * 0.3 + 0.01 + 0.6 * (b0[0, :na] > np.median(b0[0, :na]))
          + 0.3 * (b0[3, :na] % 2)).astype(np.float32)
    gc, hc, _ = binary_gh(nc_, seed=42)
    g = np.concatenate([ga, -ga, gc]).astype(np.float32)
    h = np.concatenate([ha, ha, hc]).astype(np.float32)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)
    _, dg, dh = be.discretize_dequantize_in_place(4, False, 0, want_values=True)
    og, oh, _, _ = oracle.quantize(g, h, bins=4, stochastic=False, seed=0)
    assert np.array_equal(bits(dg), bits(og))
    assert np.array_equal(dg[na:2 * na], -dg[:na])  # values: q = 0 dequantizes to +0.0
    cfg = GainConfig.make(min_data_in_leaf=20)
    t, lay = be.grow_tree_on_device_with_cfg(cfg, 63, -1)
    o, olay = oracle.train_tree(bins, meta, ub, og, oh, cfg, 63, -1)
    _compare_trees(t, o, "tied")
    assert np.array_equal(lay["indices"], olay["indices"])
    gains = t["split_gain"][: t["num_leaves"] - 1]
    say(f"  leaves {t['num_leaves']}, splits {len(gains)}, distinct gains {len(np.unique(gains))}")
    assert t["split_feature"][0] == 0
    assert len(gains) - len(np.unique(gains)) >= 10, "expected twin splits with equal gains"


# ---------------------------------------------------------------------------
# f32 gradients (use_quantized_grad = false).  Parity bar: histograms and leaf values
# within 1e-5 relative of the reference's f64 fold (the 64-bit fixed-point build is
# within ~1e-10); tree structure and partitions identical on these inputs.
# ---------------------------------------------------------------------------
def _auc(y, s):
    """ROC AUC by the rank-sum (Mann-Whitney) formula, average ranks for ties."""
    order = np.argsort(s, kind="mergesort")
    ranks = np.empty(len(s), np.float64)
    ss = s[order]
    i = 0
    while i < len(ss):
        j = i
        while j + 1 < len(ss) and ss[j + 1] == ss[i]:
            j += 1
        ranks[order[i:j + 1]] = 0.5 * (i + j) + 1.0
        i = j + 1
    pos = y > 0
    npos, nneg = pos.sum(), (~pos).sum()
    return (ranks[pos].sum() - npos * (npos + 1) / 2.0) / (npos * nneg)


@pytest.mark.parametrize("n,F,max_bin", [(40_000, 28, 255), (300_000, 13, 64)])
def test_fp32_leaf_histogram_vs_f64_fold(be, n, F, max_bin):
    say(f"fp32 leaf histogram n={n} F={F} max_bin={max_bin}")
    bins, meta, ub = make_binned(n, F, seed=F + 100, max_bin=max_bin)
    g, h, _ = binary_gh(n, seed=6)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)  # not quantized: f32 gradients
    rows = np.sort(np.random.default_rng(2).choice(n, size=n // 3, replace=False)).astype(np.uint32)
    sg = float(np.sum(g[rows].astype(np.float64)))
    sh = float(np.sum(h[rows].astype(np.float64)))
    got = be.build_resident_leaf(rows, sg, sh)
    offs, _ = slot_layout(meta)
    gabs = float(np.abs(g[rows].astype(np.float64)).sum())
    for f, m in enumerate(meta):
        hist = oracle.construct_histogram(bins[f][rows], g[rows], h[rows], m.num_bin)
        hist = oracle.fix_histogram(hist, m.num_bin, m.most_freq_bin, sg, sh)
        hist = oracle.compact_histogram(hist, m.num_bin, m.offset)
        np.testing.assert_allclose(got[offs[f]:offs[f] + 2 * m.num_bin], hist, rtol=1e-5,
                                   atol=1e-9 * gabs, err_msg=f"feature {f}")


@pytest.mark.parametrize("n,F,nl,max_bin,seed", [(100_000, 28, 31, 255, 7), (60_000, 9, 63, 64, 8)])
def test_fp32_grow_tree_vs_oracle(be, n, F, nl, max_bin, seed):
    say(f"fp32 grow_tree n={n} F={F} num_leaves={nl} max_bin={max_bin}")
    bins, meta, ub = make_binned(n, F, seed=seed, max_bin=max_bin)
    g, h, _ = binary_gh(n, seed=seed)
    be.upload_resident_bins(bins, meta, ub)
    be.upload_resident_grad_hess(g, h)
    cfg = GainConfig.make(min_data_in_leaf=20)
    t, lay = be.grow_tree_on_device_with_cfg(cfg, nl, -1)
    o, olay = oracle.train_tree(bins, meta, ub, g, h, cfg, nl, -1)
    assert t["num_leaves"] == o["num_leaves"]
    for k in ("split_feature", "threshold_in_bin", "left_child", "right_child", "leaf_count",
              "internal_count", "decision_type", "leaf_depth", "leaf_parent"):
        assert np.array_equal(t[k], o[k]), k
    for k in ("leaf_value", "internal_value", "leaf_weight", "threshold"):
        np.testing.assert_allclose(t[k], o[k], rtol=1e-5, atol=1e-12, err_msg=k)
    np.testing.assert_allclose(t["split_gain"], o["split_gain"], rtol=1e-5, err_msg="split_gain")
    assert np.array_equal(lay["indices"], olay["indices"])


def test_fp32_train_binary_config0_auc():
    """BASELINE configs[0] (100k x 28 ~N(0,1), max_bin 255, f32 gradients, num_leaves
    31, all 100 iterations): every tree's structure identical to the oracle's, leaf
    values within 1e-5 relative, training scores within 1e-6 and the final AUC within
    1e-6 of the oracle's."""
    from lightgbm_rs_amd.synth import config0_like
    n, iters, nl = 100_000, 100, 31
    bins, meta, ub, y = config0_like(n)
    init = oracle.boost_from_score(y)
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.set_labels(y, init)
        cfg = GainConfig.make(min_data_in_leaf=20)
        trees = [b.train_iter_binary(i, cfg, nl, -1, 0.1, 0, False) for i in range(iters)]
        scores = b.scores()
    finally:
        b.close()
    oscores, otrees = oracle.train_binary(bins, meta, ub, y, cfg, nl, -1, iters, 0.1,
                                          quantized=False)
    assert len(trees) == len(otrees) == iters
    for i, (t, o) in enumerate(zip(trees, otrees)):
        assert t["num_leaves"] == o["num_leaves"], i
        for k in ("split_feature", "threshold_in_bin", "decision_type", "left_child",
                  "right_child", "leaf_count", "internal_count", "leaf_depth", "leaf_parent"):
            assert np.array_equal(t[k], o[k]), (i, k)
        lv = t["leaf_value"] if i else _mrz(t["leaf_value"] + init)
        np.testing.assert_allclose(lv, o["leaf_value"], rtol=1e-5, atol=1e-12, err_msg=str(i))
    np.testing.assert_allclose(scores, oscores, rtol=0, atol=1e-6)
    a, oa = _auc(y, scores), _auc(y, oscores)
    say(f"  AUC {a:.9f} oracle {oa:.9f}")
    assert abs(a - oa) <= 1e-6


@pytest.mark.parametrize("qbins", [4, 0])
def test_lookahead_matches_plain_iterations(qbins):
    """lgbm_hip_set_lookahead: the next iteration's gradients and quantization run
    while the host reads the tree; trees and scores are bit-identical to the plain
    loop, also across an invalidating call (set_labels) and a skipped iteration."""
    from lightgbm_rs_amd import binary_boost_from_score
    n = 60_000
    bins, meta, ub, y = config1_like(n, seed=13)
    init = binary_boost_from_score(y)
    cfg = GainConfig.make(min_data_in_leaf=20)
    runs = []
    for look in (False, True):
        b = HipBackend(0)
        try:
            b.upload_resident_bins(bins, meta, ub)
            b.set_labels(y, init)
            b.set_lookahead(look)
            trees = [b.train_iter_binary(i, cfg, 63, -1, 0.1, qbins, True) for i in range(3)]
            b.set_labels(y, init)  # drops a pending lookahead
            trees += [b.train_iter_binary(i, cfg, 63, -1, 0.1, qbins, True) for i in (0, 1, 5, 6)]
            runs.append((trees, b.scores()))
        finally:
            b.close()
    (ta, sa), (tb, sb) = runs
    for i, (x, z) in enumerate(zip(ta, tb)):
        _compare_trees(x, z, f"iteration {i}")
    assert np.array_equal(bits(sa), bits(sb))
