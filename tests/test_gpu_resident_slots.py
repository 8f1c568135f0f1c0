"""The device-resident slot seam (Backend::reset_resident_pool / build_resident_leaf /
move_resident / subtract_resident / scan_resident_leaf / scan_resident_siblings,
crates/lgbm-compute/src/lib.rs:1940-2058) driven by a host learner loop.

The loop below is SerialTreeLearner::train_inner's resident arm (learner.rs:980-1562,
1808-1839 gates, 1851-2453 find_best_splits with the smaller-child build and the
subtraction, 4537 ArgMax, 3895-4092 split_inner with partition counts): every leaf
histogram stays in a device slot, only SplitInfos come back, and rows are split by the
per-op DataPartition.  A 255-leaf tree grown this way must equal lgbm_hip_grow_tree's
(the whole-tree seam) bit for bit, and the slot histograms must equal the host-returning
per-op build.
"""
import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend
from lightgbm_rs_amd._abi import BatchedFeature
from tests.datagen import config1_like, make_binned

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _batched(meta):
    out, off = [], 0
    for m in meta:
        nb, mt = int(m.num_bin), int(m.missing_type)
        out.append(BatchedFeature(off, nb, int(m.offset), int(m.default_bin), int(m.most_freq_bin),
                                  int(nb > 2 and mt == 1), int(nb > 2 and mt == 2),
                                  int(nb > 2 and mt != 0), 0))
        off += 2 * nb
    return out


def _split_gt(a, fa, b, fb):
    """split_gt (split_info.rs:28-35): higher gain, then lower real feature (-1 last)."""
    if a.gain != b.gain:
        return a.gain > b.gain
    big = 2 ** 31 - 1
    return (big if fa == -1 else fa) < (big if fb == -1 else fb)


class _NoSplit:
    gain = -np.inf


def grow_resident(be, bins, meta, cfg, num_leaves, sg, sh):
    """The host learner loop over the resident slots; returns the tree's arrays."""
    F, N = bins.shape
    feats = _batched(meta)
    real = [int(m.real_feature_index) for m in meta]
    tmp = num_leaves  # the parent's histogram while its children take their slots
    be.reset_resident_pool(num_leaves + 1)
    rows = {0: np.arange(N, dtype=np.uint32)}
    root_w = -sg / (sh + cfg.lambda_l2)
    T = dict(split_feature=[], threshold_in_bin=[], split_gain=[], internal_value=[],
             internal_count=[], internal_weight=[], left_child=[], right_child=[], decision_type=[],
             leaf_value=[root_w], leaf_weight=[0.0], leaf_count=[N], leaf_depth=[0], leaf_parent=[-1])
    best = [_NoSplit()] * num_leaves
    best_feat = [-1] * num_leaves
    splittable = {0: np.ones(F, bool)}
    smaller, larger = (N, sg, sh, root_w), None
    left_leaf, right_leaf = 0, -1
    min2 = cfg.min_data_in_leaf * 2

    def scan_into(leaf, si, scanned):
        this = np.zeros(F, bool)
        lb, lbf = _NoSplit(), -1
        for f, s in zip(scanned, si):
            this[f] = s.gain > -np.inf
            if s.gain > -np.inf and _split_gt(s, real[f], lb, lbf):
                lb, lbf = s, real[f]
        best[leaf], best_feat[leaf] = lb, lbf
        splittable[leaf] = this

    for _ in range(num_leaves - 1):
        # before_find_best_split
        did = True
        if right_leaf >= 0 and len(rows[right_leaf]) < min2 and len(rows[left_leaf]) < min2:
            did = False
        elif right_leaf < 0 and len(rows[left_leaf]) < min2:
            did = False
        if not did:
            best[left_leaf] = _NoSplit()
            if right_leaf >= 0:
                best[right_leaf] = _NoSplit()
        else:
            if right_leaf < 0:
                sm, lg, s_ls, l_ls = left_leaf, -1, smaller, None
            elif len(rows[left_leaf]) < len(rows[right_leaf]):
                sm, lg = left_leaf, right_leaf
                s_ls, l_ls = smaller, larger
            else:
                sm, lg = right_leaf, left_leaf
                s_ls, l_ls = smaller, larger
            use_sub = right_leaf >= 0
            parent_split = splittable[left_leaf] if use_sub else np.ones(F, bool)
            if use_sub:
                be.move_resident(left_leaf, tmp)
            assert s_ls[2] > 0.0 and s_ls[0] > 0
            be.build_resident_leaf(rows[sm], s_ls[1], s_ls[2], slot=sm)
            if lg >= 0:
                be.subtract_resident(tmp, sm, lg)
            scanned = [f for f in range(F) if parent_split[f]]
            fs = [feats[f] for f in scanned]
            if lg >= 0:
                assert l_ls[2] > 0.0 and l_ls[0] > 0
                tot = lambda ls: (ls[1], ls[2], ls[0], ls[3])  # noqa: E731
                if fs:
                    a, b = be.scan_resident_siblings(sm, lg, fs, cfg, tot(s_ls), tot(l_ls))
                else:
                    a, b = [], []
                scan_into(sm, a, scanned)
                scan_into(lg, b, scanned)
            else:
                c = GainConfig.from_buffer_copy(cfg)
                c.parent_output = s_ls[3]
                scan_into(sm, be.scan_resident_leaf(sm, fs, c, s_ls[1], s_ls[2], s_ls[0]), scanned)
        # ArgMax over the leaves (first max wins)
        bl = 0
        for i in range(1, num_leaves):
            if _split_gt(best[i], best_feat[i], best[bl], best_feat[bl]):
                bl = i
        b = best[bl]
        if not (b.gain > 0.0):
            break
        f = real.index(best_feat[bl])
        m = meta[f]
        new_right = len(T["leaf_value"])
        r = rows[bl]
        pmin = int(m.min_bin) + max(int(m.offset), 0)
        order, lc = be.data_partition(bins[f][r], int(m.num_bin), pmin, int(m.max_bin), b.threshold,
                                      int(m.most_freq_bin),
                                      int(m.num_bin) > 2 and int(m.missing_type) == 2,
                                      bool(b.default_left))
        rows[bl], rows[new_right] = r[order[:lc]], r[order[lc:]]
        pl, pr = int(lc), len(r) - int(lc)
        # Tree::split (tree.rs:614-700)
        node = new_right - 1
        parent = T["leaf_parent"][bl]
        if parent >= 0:
            if T["right_child"][parent] == ~bl:
                T["right_child"][parent] = node
            else:
                T["left_child"][parent] = node
        T["split_feature"].append(best_feat[bl])
        T["split_gain"].append(np.float32(b.gain + cfg.min_gain_to_split))
        T["threshold_in_bin"].append(b.threshold)
        T["internal_value"].append(T["leaf_value"][bl])
        T["internal_count"].append(pl + pr)
        T["internal_weight"].append(b.left_sum_hessian + b.right_sum_hessian)
        T["left_child"].append(~bl)
        T["right_child"].append(~new_right)
        T["decision_type"].append((2 if b.default_left else 0) | ((int(m.missing_type) & 3) << 2))
        T["leaf_value"][bl] = b.left_output
        T["leaf_weight"][bl] = b.left_sum_hessian
        T["leaf_count"][bl] = pl
        T["leaf_value"].append(b.right_output)
        T["leaf_weight"].append(b.right_sum_hessian)
        T["leaf_count"].append(pr)
        T["leaf_depth"].append(T["leaf_depth"][bl] + 1)
        T["leaf_depth"][bl] += 1
        T["leaf_parent"][bl] = node
        T["leaf_parent"].append(node)
        # child seeding by partition counts (learner.rs:4061)
        lsd = (pl, b.left_sum_gradient, b.left_sum_hessian, b.left_output)
        rsd = (pr, b.right_sum_gradient, b.right_sum_hessian, b.right_output)
        smaller, larger = (lsd, rsd) if pl < pr else (rsd, lsd)
        for leaf in (bl, new_right):
            best[leaf], best_feat[leaf] = _NoSplit(), -1
        left_leaf, right_leaf = bl, new_right
    T["num_leaves"] = len(T["leaf_value"])
    return T, rows


@pytest.mark.parametrize("kind,n,nl,seed", [("config1", 200_000, 255, 21),
                                             ("mixed", 60_000, 255, 22),
                                             ("config1", 30_000, 63, 23)])
def test_resident_slots_grow_the_whole_tree_seams_tree(kind, n, nl, seed):
    """kind config1: configs[1]'s features; mixed: bin counts of 2-64, most frequent
    bins (FixHistogram), missing types Zero / NaN (skip-default-bin, FORWARD scans,
    NaN routing)."""
    if kind == "config1":
        bins, meta, ub, _ = config1_like(n, seed=seed)
    else:
        bins, meta, ub = make_binned(n, 24, seed=seed)
    say(f"resident slots {kind} n={n} num_leaves={nl}")
    rng = np.random.default_rng(seed)
    s = rng.normal(0, 1, n)
    p = 1 / (1 + np.exp(-s))
    y = (rng.random(n) < p).astype(np.float32)
    g = (p - y).astype(np.float32)
    h = (p * (1 - p)).astype(np.float32)
    cfg = GainConfig.make(min_data_in_leaf=20)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, ub)
        be.upload_resident_grad_hess(g, h)
        _, dg, dh = be.discretize_dequantize_in_place(4, True, 0x51702010, want_values=True)
        # quantized values: every partial sum is exact, so any summation order gives
        # the ordered f64 fold's root totals
        sg = float(np.sum(dg.astype(np.float64)))
        sh = float(np.sum(dh.astype(np.float64)))
        want, lay = be.grow_tree_on_device_with_cfg(cfg, nl, -1)
        say(f"whole-tree seam: {want['num_leaves']} leaves")
        got, rows = grow_resident(be, bins, meta, cfg, nl, sg, sh)
        say(f"resident slots: {got['num_leaves']} leaves")
        # a slot equals the host-returning per-op build of the same leaf
        leaf = int(np.argmax(got["leaf_count"]))
        r = rows[leaf]
        lsg = float(np.sum(dg[r].astype(np.float64)))
        lsh = float(np.sum(dh[r].astype(np.float64)))
        be.build_resident_leaf(r, lsg, lsh, slot=0)
        host = be.build_resident_leaf(r, lsg, lsh)
        assert np.array_equal(be.read_resident(0).view(np.uint64), host.view(np.uint64))
    finally:
        be.close()
    assert got["num_leaves"] == want["num_leaves"]
    for k in ("split_feature", "threshold_in_bin", "left_child", "right_child", "leaf_count",
              "internal_count", "leaf_depth", "leaf_parent", "decision_type"):
        assert np.array_equal(np.asarray(got[k]), np.asarray(want[k])), k
    for k in ("leaf_value", "leaf_weight", "internal_value", "internal_weight"):
        a = np.asarray(got[k], np.float64).view(np.uint64)
        b = np.asarray(want[k], np.float64).view(np.uint64)
        assert np.array_equal(a, b), k
    assert np.array_equal(np.asarray(got["split_gain"], np.float32),
                          np.asarray(want["split_gain"], np.float32))
    # each leaf's rows are the layout's (ascending in both)
    for leaf in range(got["num_leaves"]):
        b0, c0 = int(lay["leaf_begin"][leaf]), int(lay["leaf_count"][leaf])
        assert np.array_equal(rows[leaf], lay["indices"][b0:b0 + c0]), leaf


def test_resident_slot_errors():
    bins, meta, ub, _ = config1_like(5000, seed=3)
    be = HipBackend(0)
    try:
        be.upload_resident_bins(bins, meta, ub)
        with pytest.raises(Exception, match="reset the resident pool"):
            be.move_resident(0, 1)
        with pytest.raises(Exception, match="LENGTH_MISMATCH"):
            be.reset_resident_pool(4, be.slot_len + 2)
        be.reset_resident_pool(4)
        with pytest.raises(Exception, match="outside"):
            be.subtract_resident(0, 1, 4)
        with pytest.raises(Exception, match="coincide"):
            be.subtract_resident(0, 1, 1)
        # a new bins upload invalidates the pool
        be.upload_resident_bins(bins[:20], meta[:20], ub[:sum(int(m.num_bin) for m in meta[:20])])
        with pytest.raises(Exception, match="predates"):
            be.move_resident(0, 1)
    finally:
        be.close()
