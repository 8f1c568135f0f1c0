"""The reference's real-binary goldens replayed on the device (the same fixtures that
pin the oracle in test_oracle_golden.py), plus the quantizer seam and feature_contri
through the C-ABI.

  * learner_real.json: real lib_lightgbm 4.6 trees (learner_parity.rs:1214/1297,
    na_missing_parity.rs:193, gain_params_parity.rs:170-226) grown by
    lgbm_hip_grow_tree from the same f32 gradients: every learner field bit-exact.
  * path_smooth.npz: 13 (path_smooth, max_delta_step, lambda_l1, num_leaves) boosting
    runs of the real binary (path_smooth_parity.rs:274-345) through
    lgbm_hip_train_iter_binary with f32 gradients: leaf values and training scores
    bit-exact (the reference's own gate is 1e-6 as f32).
  * lgbm_hip_set_dequantized_gradients: the q recovered from dequantized values grows
    the same tree as the device quantizer's own q; altered values are refused.
"""
import os

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend, binary_boost_from_score, feature_mappers
from lightgbm_rs_amd.backend import HipError
from oracle import oracle
from tests.datagen import binary_gh, make_binned
from tests.test_oracle_golden import (assert_real_tree, learner_case_inputs, load,
                                      path_smooth_cells)

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


@pytest.mark.parametrize("case", load("learner_real.json"), ids=lambda c: c["name"])
def test_learner_real_tree_on_device(be, case):
    say("learner_real on device", case["name"])
    bins, meta, upper, cfg, contri = learner_case_inputs(case)
    be.upload_resident_bins(bins.astype(np.uint8), meta, upper)
    if contri is not None:
        be.set_feature_contri(contri)
    be.upload_resident_grad_hess(np.array(case["grad"], np.float32),
                                 np.array(case["hess"], np.float32))
    t, lay = be.grow_tree_on_device_with_cfg(cfg, case["num_leaves"], case["max_depth"])
    assert_real_tree(t, case)
    o, olay = oracle.train_tree(bins, meta, upper, case["grad"], case["hess"], cfg,
                                case["num_leaves"], case["max_depth"], feature_contri=contri)
    assert np.array_equal(lay["indices"], olay["indices"])
    assert np.array_equal(t["split_gain"], o["split_gain"])


def _mrz(v):
    z = float(np.float32(1e-35))
    return np.where((v >= -z) & (v <= z), 0.0, v)


@pytest.mark.parametrize("cell", range(13))
def test_path_smooth_cells_on_device(be, cell):
    z = np.load(os.path.join(GOLD, "path_smooth.npz"))
    c = path_smooth_cells()[cell]
    say("path_smooth cell on device", cell, c["ps"], c["mds"], c["l1"], c["nl"])
    X, y = z["X"], z["y"].astype(np.float32)
    ms = feature_mappers(X, max_bin=63, min_data_in_leaf=5)
    init = binary_boost_from_score(y)
    be.upload_raw(X, ms)
    be.set_labels(y, init)
    cfg = GainConfig.make(min_data_in_leaf=5, lambda_l1=c["l1"], max_delta_step=c["mds"],
                          path_smooth=c["ps"])
    for i in range(int(z["num_iterations"])):
        t = be.train_iter_binary(i, cfg, c["nl"], -1, 0.1, 0, False)
        lv = t["leaf_value"][:t["num_leaves"]]
        if i == 0:
            lv = _mrz(lv + init)  # Tree::add_bias of the first iteration (tree.rs:1161)
        gold = np.ascontiguousarray(c["leaves"][i])
        assert len(lv) == len(gold), i
        assert np.array_equal(lv.view(np.uint64), gold.view(np.uint64)), (i, lv - gold)
    scores = be.scores()
    assert np.array_equal(scores.view(np.uint64), np.ascontiguousarray(c["pred"]).view(np.uint64))


def test_dequantized_seam_grows_the_quantizer_tree():
    """The drop-in wiring at gbdt.rs:945-960: the device quantizes the raw gradients
    (writing f32(q * scale) back like discretize_dequantize_in_place), the learner
    uploads those values, and the device recovers q from them — the same tree as
    the device's own q, with the context's scales or the scales passed in."""
    n, F, nl = 200_000, 9, 63
    say("dequantized seam", n, F, nl)
    bins, meta, ub = make_binned(n, F, seed=71)
    g, h, _ = binary_gh(n, seed=71)
    cfg = GainConfig.make(min_data_in_leaf=20)
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.upload_resident_grad_hess(g, h)
        scales, dg, dh = b.discretize_dequantize_in_place(4, True, 0x51702010 ^ (3 << 20),
                                                          want_values=True)
        disc = b.discretized()
        t0, l0 = b.grow_tree_on_device_with_cfg(cfg, nl, -1)
        b.set_dequantized_grad_hess(dg, dh, 4)  # the context's scales
        assert np.array_equal(b.discretized(), disc)
        t1, l1 = b.grow_tree_on_device_with_cfg(cfg, nl, -1)
        b.upload_resident_grad_hess(g, h)  # raw values again, then explicit scales
        b.set_dequantized_grad_hess(dg, dh, 4, scales[0], scales[1])
        assert np.array_equal(b.discretized(), disc)
        t2, l2 = b.grow_tree_on_device_with_cfg(cfg, nl, -1)
        for t, lay in ((t1, l1), (t2, l2)):
            for k in ("split_feature", "threshold_in_bin", "leaf_count", "left_child",
                      "right_child"):
                assert np.array_equal(t[k], t0[k]), k
            for k in ("leaf_value", "leaf_weight", "internal_value"):
                assert np.array_equal(t[k].view(np.uint64), t0[k].view(np.uint64)), k
            assert np.array_equal(lay["indices"], l0["indices"])
        # altered values are refused and leave no gradients to grow from
        bad = dh.copy()
        bad[17] = np.nextafter(bad[17], np.float32(1.0))
        with pytest.raises(HipError, match="first row 17"):
            b.set_dequantized_grad_hess(dg, bad, 4)
        with pytest.raises(HipError):
            b.grow_tree_on_device_with_cfg(cfg, nl, -1)
    finally:
        b.close()


def test_failed_reupload_leaves_no_usable_state():
    """A bins upload that fails inside the resident setup leaves the context without
    bins, gradients or a replayable tree graph (the next calls return errors)."""
    n, F = 50_000, 7
    say("failed re-upload", n, F)
    bins, meta, ub = make_binned(n, F, seed=81)
    g, h, _ = binary_gh(n, seed=81)
    cfg = GainConfig.make(min_data_in_leaf=20)
    b = HipBackend(0)
    try:
        b.upload_resident_bins(bins, meta, ub)
        b.upload_resident_grad_hess(g, h)
        b.discretize_dequantize_in_place(4, True, 1)
        b.grow_tree_on_device_with_cfg(cfg, 31, -1)  # captures the tree graph
        # 4097 features: more than any row layout holds (WIDE_MAX_F)
        wide, wmeta, wub = make_binned(64, 4097, seed=82, max_bin=4, missing_mix=False,
                                       mfb_mix=False)
        with pytest.raises(HipError):
            b.upload_resident_bins(wide, wmeta, wub)
        with pytest.raises(HipError):
            b.grow_tree_on_device_with_cfg(cfg, 31, -1)
        with pytest.raises(HipError):
            b.upload_resident_grad_hess(g, h)
        # and a valid upload makes it usable again
        b.upload_resident_bins(bins, meta, ub)
        b.upload_resident_grad_hess(g, h)
        b.discretize_dequantize_in_place(4, True, 1)
        t, _ = b.grow_tree_on_device_with_cfg(cfg, 31, -1)
        assert t["num_leaves"] == 31
    finally:
        b.close()
