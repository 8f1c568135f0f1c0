"""Pin the CPU oracle against the reference's own golden vectors (CPU only).

Each test names the reference test whose semantics it replays.  Fixtures are the
reference's committed golden files re-encoded by tests/golden/make_golden.py.
"""
import json
import os
import struct

import numpy as np
import pytest

from lightgbm_rs_amd._abi import FeatureMeta, GainConfig
from oracle import oracle

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def f32(bits):
    return np.array(bits, dtype=np.uint32).view(np.float32)


def f64(bits):
    return np.array(bits, dtype=np.uint64).view(np.float64)


def b64(x):
    return struct.unpack("<Q", struct.pack("<d", float(x)))[0]


# --- kernel_parity.rs:162 (histogram bit-exact) -------------------------------
@pytest.mark.parametrize("case", load("hist_f64.json"), ids=lambda c: c["name"])
def test_histogram_fold_bit_exact(case):
    got = oracle.construct_histogram(case["bins"], f32(case["grad_bits"]), f32(case["hess_bits"]),
                                     case["num_bin"])
    exp = np.zeros(case["hist_len"], dtype=np.uint64)
    for k, v in case["hist_nonzero_bits"]:
        exp[k] = v
    assert np.array_equal(got.view(np.uint64), exp)


# --- kernel_parity.rs:512 (split winner bit-exact) -----------------------------
@pytest.mark.parametrize("case", load("split_scan.json"), ids=lambda c: c["name"])
def test_split_winner_bit_exact(case):
    cfg = GainConfig.make(min_data_in_leaf=case["min_data_in_leaf"],
                          min_sum_hessian_in_leaf=f64([case["min_sum_hessian_in_leaf_bits"]])[0],
                          lambda_l1=f64([case["lambda_l1_bits"]])[0],
                          lambda_l2=f64([case["lambda_l2_bits"]])[0],
                          min_gain_to_split=f64([case["min_gain_to_split_bits"]])[0])
    si = oracle.find_best_split(f64(case["hist_bits"]), cfg, case["num_bin"], case["offset"],
                                case["default_bin"], case["skip_default_bin"],
                                case["na_as_missing"], True, f64([case["sum_gradient_bits"]])[0],
                                f64([case["sum_hessian_bits"]])[0], case["num_data"])
    w = case["win"]
    assert (si.gain == -np.inf) == (not w["is_splittable"])
    if w["is_splittable"]:
        for k in ["gain", "left_sum_gradient", "left_sum_hessian", "right_sum_gradient",
                  "right_sum_hessian", "left_output", "right_output"]:
            assert b64(getattr(si, k)) == w[k + "_bits"], k
        assert si.threshold == w["threshold"]
        assert si.left_count == w["left_count"]
        assert si.right_count == w["right_count"]
        assert si.default_left == w["default_left"]


def test_split_cases_cover_both_branches():
    wins = [c["win"] for c in load("split_scan.json") if c["win"]["is_splittable"]]
    assert any(w["default_left"] for w in wins) and any(not w["default_left"] for w in wins)


# --- kernel_parity.rs:1276 (subtract bit-exact) --------------------------------
@pytest.mark.parametrize("case", load("subtract.json"), ids=lambda c: c["name"])
def test_subtract_bit_exact(case):
    got = oracle.subtract(f64(case["parent_bits"]), f64(case["child_bits"]))
    assert np.array_equal(got.view(np.uint64), np.array(case["derived_bits"], dtype=np.uint64))


# --- kernel_parity.rs:1162 (partition, missing_type == None cases) -----------
@pytest.mark.parametrize("case", [c for c in load("partition.json") if c["missing_type"] == 0],
                         ids=lambda c: c["name"])
def test_partition_exact(case):
    order, split = oracle.data_partition(case["bins"], case["num_bin"], case["min_bin"],
                                         case["max_bin"], case["threshold"],
                                         case["most_freq_bin"])
    assert order.tolist() == case["order"]
    assert split == case["split_point"]


# --- real lib_lightgbm 4.6 trees: learner_parity.rs:1214 / 1297,
#     na_missing_parity.rs:193 (NaN FORWARD preamble + NaN routing),
#     gain_params_parity.rs:170-226 (feature_contri, max_delta_step, path_smooth) -----
def _maybe_round_to_zero(v):
    z = float(np.float32(1e-35))
    return 0.0 if -z <= v <= z else v


def learner_case_inputs(case):
    """(bins, meta, upper, cfg, feature_contri) of a learner_real.json corpus."""
    nb = case["num_bin"]
    meta = [FeatureMeta(nb, 1 if case["most_freq_bin"] == 0 else 0, 0, nb - 1,
                        case.get("default_bin", nb), case["most_freq_bin"],
                        case.get("missing_type", 0), 0, case.get("bin_type", 0))]
    bins = np.array([case["bins"]], dtype=np.uint32)
    cfg = GainConfig.make(min_data_in_leaf=case["min_data_in_leaf"],
                          min_sum_hessian_in_leaf=case["min_sum_hessian_in_leaf"],
                          max_delta_step=case.get("max_delta_step", 0.0),
                          path_smooth=case.get("path_smooth", 0.0))
    for k, v in case.get("cat", {}).items():
        setattr(cfg, k, v)
    return bins, meta, f64(case["upper_bits"]), cfg, case.get("feature_contri")


def assert_real_tree(t, case):
    """Every learner-authoritative field of the real binary's Tree=0 block."""
    g = case["tree"]
    assert t["num_leaves"] == int(g["num_leaves"][0])
    assert t["split_feature"].tolist() == [int(x) for x in g["split_feature"]]
    assert t["decision_type"].tolist() == [int(x) for x in g["decision_type"]]
    assert t["left_child"].tolist() == [int(x) for x in g["left_child"]]
    assert t["right_child"].tolist() == [int(x) for x in g["right_child"]]
    assert t["leaf_count"].tolist() == [int(x) for x in g["leaf_count"]]
    assert t["internal_count"].tolist() == [int(x) for x in g["internal_count"]]
    assert [b64(x) for x in t["threshold"]] == [b64(float(x)) for x in g["threshold"]]
    shrunk = [_maybe_round_to_zero(v * case["shrinkage"]) for v in t["leaf_value"]]
    assert [b64(x) for x in shrunk] == [b64(float(x)) for x in g["leaf_value"]]
    # categorical splits: the real-category bitsets (Tree::split_categorical)
    assert t["num_cat"] == int(g.get("num_cat", ["0"])[0])
    if t["num_cat"]:
        assert t["cat_boundaries"].tolist() == [int(x) for x in g["cat_boundaries"]]
        assert t["cat_threshold"].tolist() == [int(x) for x in g["cat_threshold"]]
    if case.get("check_split_gain"):
        # split_gain is f32 in the model and %g in the text (gain_params_parity.rs:151-158)
        assert ["%g" % np.float32(x) for x in t["split_gain"]] == [
            "%g" % float(x) for x in g["split_gain"]]


@pytest.mark.parametrize("case", load("learner_real.json"), ids=lambda c: c["name"])
def test_learner_real_tree(case):
    bins, meta, upper, cfg, contri = learner_case_inputs(case)
    t, layout = oracle.train_tree(bins, meta, upper, case["grad"], case["hess"], cfg,
                                  case["num_leaves"], case["max_depth"], feature_contri=contri)
    assert_real_tree(t, case)
    # partition layout is a permutation consistent with the leaf counts
    assert sorted(layout["indices"].tolist()) == list(range(len(case["grad"])))
    assert layout["leaf_count"].tolist() == t["leaf_count"].tolist()


# --- gradient_discretizer.rs:269-333 (hand-computed cases) --------------------
@pytest.mark.parametrize("case", load("discretizer_cases.json"), ids=lambda c: c["name"])
def test_discretizer_hand_cases(case):
    g, h, disc, scales = oracle.quantize(case["grad"], case["hess"], bins=case["bins"],
                                         stochastic=False, const_hess=case["const_hess"])
    qg, qh = disc[1::2].tolist(), disc[0::2].tolist()
    if "grad_scale" in case:
        assert scales[0] == case["grad_scale"]
    if "hess_scale" in case:
        assert scales[1] == case["hess_scale"]
    if "q_grad" in case:
        assert qg == case["q_grad"]
    if "q_hess" in case:
        assert qh == case["q_hess"]
    for k, v in case.get("q_grad_sel", {}).items():
        assert qg[int(k)] == v
    if "int_hist" in case:
        ih = oracle.int_histogram(case["binned"], disc, np.arange(len(case["grad"])),
                                  case["num_bin"])
        assert ih.tolist() == case["int_hist"]
    # dequantized write-back is f32(q * scale) (gradient_discretizer.rs:136-137)
    assert np.array_equal(g, (np.array(qg, np.float64) * scales[0]).astype(np.float32))


def test_stochastic_reproducible_and_seed_dependent():
    # gradient_discretizer.rs:337-346
    grad = (np.arange(200, dtype=np.float32) - 100.0) * np.float32(0.013)
    hess = np.ones(200, np.float32)
    a = oracle.quantize(grad, hess, bins=16, stochastic=True, seed=42, const_hess=1)[2]
    b = oracle.quantize(grad, hess, bins=16, stochastic=True, seed=42, const_hess=1)[2]
    c = oracle.quantize(grad, hess, bins=16, stochastic=True, seed=43, const_hess=1)[2]
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)


def test_stochastic_rounding_unbiased():
    # gradient_discretizer.rs:348-376: deterministic rounds the off-grid bulk to the
    # grid point, stochastic rounding averages back to the true value.
    n = 20002
    grad = np.full(n, 0.3, np.float32)
    grad[0], grad[1] = 1.0, -1.0
    hess = np.ones(n, np.float32)
    _, _, qd, sd = oracle.quantize(grad, hess, bins=4, stochastic=False, const_hess=1)
    _, _, qs, ss = oracle.quantize(grad, hess, bins=4, stochastic=True, seed=7, const_hess=1)
    det = qd[1::2][2:].astype(np.int64).sum() * sd[0] / (n - 2)
    sto = qs[1::2][2:].astype(np.int64).sum() * ss[0] / (n - 2)
    assert abs(det - 0.5) < 1e-9
    assert abs(sto - 0.3) < 0.01


def test_xorshift_uniform_and_period_structure():
    # next_u01 (gradient_discretizer.rs:255-263) maps the top 53 bits to [0,1): values
    # lie on the 2^-53 grid, are in range, and the stream is uniform.
    u = oracle.xorshift_u01(0x9E3779B97F4A7C15 ^ 42, 200000)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert np.all(u * 2.0 ** 53 == np.floor(u * 2.0 ** 53))
    assert abs(u.mean() - 0.5) < 0.005
    assert abs((u < 0.25).mean() - 0.25) < 0.005
    # a jump of k steps equals k single steps: state after 3 draws restarts the tail
    v = oracle.xorshift_u01(0x9E3779B97F4A7C15 ^ 42, 3)
    assert np.array_equal(v, u[:3])


def test_learner_real_cases_have_teeth():
    """Each gain option's golden differs from the plain-gain tree: a learner that
    ignored feature_contri / max_delta_step / path_smooth would fail its case."""
    cases = {c["name"]: c for c in load("learner_real.json")}
    plain = dict(cases["gain_params_penalty"])
    plain.pop("feature_contri")
    bins, meta, upper, cfg, _ = learner_case_inputs(plain)
    t, _ = oracle.train_tree(bins, meta, upper, plain["grad"], plain["hess"], cfg, 2, -1)
    for name in ("gain_params_penalty", "gain_params_max_delta_step", "gain_params_path_smooth"):
        g = cases[name]["tree"]
        differs = (np.float32(t["split_gain"][0]) != np.float32(float(g["split_gain"][0])) or
                   any(b64(_maybe_round_to_zero(v * 0.1)) != b64(float(x))
                       for v, x in zip(t["leaf_value"], g["leaf_value"])))
        assert differs, name
    # the NaN corpus with missing type None grows a different tree than the real binary
    na = dict(cases["na_missing_real"], missing_type=0)
    bins, meta, upper, cfg, _ = learner_case_inputs(na)
    t, _ = oracle.train_tree(bins, meta, upper, na["grad"], na["hess"], cfg, 2, -1)
    g = cases["na_missing_real"]["tree"]
    assert (t["decision_type"].tolist() != [int(x) for x in g["decision_type"]] or
            t["leaf_count"].tolist() != [int(x) for x in g["leaf_count"]])


def _real_tree_fails(case):
    bins, meta, upper, cfg, contri = learner_case_inputs(case)
    t, _ = oracle.train_tree(bins, meta, upper, case["grad"], case["hess"], cfg,
                             case["num_leaves"], case["max_depth"], feature_contri=contri)
    try:
        assert_real_tree(t, case)
    except AssertionError:
        return True
    return False


def test_categorical_cases_have_teeth():
    """The categorical goldens tell apart the scan's options: one-hot in place of
    many-vs-many, a dropped cat_l2, a different cat_smooth, and the feature taken as numerical
    each fail a case."""
    cases = {c["name"]: c for c in load("learner_real.json")}
    mvm, onehot = cases["cat_manyvsmany_real"], cases["cat_onehot_real"]
    assert not _real_tree_fails(mvm) and not _real_tree_fails(onehot)
    assert _real_tree_fails(dict(mvm, cat=dict(mvm["cat"], max_cat_to_onehot=64)))
    assert _real_tree_fails(dict(onehot, cat=dict(onehot["cat"], cat_l2=0.0)))
    # cat_smooth both smooths the sort key and drops categories with fewer rows
    assert _real_tree_fails(dict(mvm, cat=dict(mvm["cat"], cat_smooth=11.0)))
    assert _real_tree_fails(dict(mvm, bin_type=0))


# --- kernel_parity.rs:240-320, 369-466 (per-candidate REVERSE / FORWARD gains) ----
def _cand_equal(got, bits_list):
    exp = f64(bits_list)
    if len(got) != len(exp):
        return False
    for a, b in zip(got, exp):
        if np.isnan(a) or np.isnan(b):
            if not (np.isnan(a) and np.isnan(b)):
                return False
        elif b64(a) != b64(b):
            return False
    return True


@pytest.mark.parametrize("case", load("split_scan.json"), ids=lambda c: c["name"])
def test_split_candidates_bit_exact(case):
    """Every candidate gain of both scan directions (NaN where gated) equals the
    golden's SCAND_REV / SCAND_FWD vectors bit for bit: the scan's prefix order, gates
    and gain arithmetic, not only its winner."""
    cfg = GainConfig.make(min_data_in_leaf=case["min_data_in_leaf"],
                          min_sum_hessian_in_leaf=f64([case["min_sum_hessian_in_leaf_bits"]])[0],
                          lambda_l1=f64([case["lambda_l1_bits"]])[0],
                          lambda_l2=f64([case["lambda_l2_bits"]])[0],
                          min_gain_to_split=f64([case["min_gain_to_split_bits"]])[0])
    rev, fwd = oracle.split_candidates(
        f64(case["hist_bits"]), cfg, case["num_bin"], case["offset"], case["default_bin"],
        case["skip_default_bin"], case["na_as_missing"], True,
        f64([case["sum_gradient_bits"]])[0], f64([case["sum_hessian_bits"]])[0],
        case["num_data"])
    assert _cand_equal(rev, case["cand_rev_bits"]), (rev, f64(case["cand_rev_bits"]))
    assert _cand_equal(fwd, case["cand_fwd_bits"]), (fwd, f64(case["cand_fwd_bits"]))


def test_split_candidates_pin_has_teeth():
    """A planted mistake fails the candidate pin: swapping the REVERSE sums' roles
    (a transposed operand) changes at least one golden vector."""
    bad = 0
    for case in load("split_scan.json"):
        h = f64(case["hist_bits"]).reshape(-1, 2)[::-1].ravel()  # bins reversed
        cfg = GainConfig.make(min_data_in_leaf=case["min_data_in_leaf"],
                              min_sum_hessian_in_leaf=f64([case["min_sum_hessian_in_leaf_bits"]])[0],
                              lambda_l1=f64([case["lambda_l1_bits"]])[0],
                              lambda_l2=f64([case["lambda_l2_bits"]])[0])
        rev, fwd = oracle.split_candidates(
            h, cfg, case["num_bin"], case["offset"], case["default_bin"],
            case["skip_default_bin"], case["na_as_missing"], True,
            f64([case["sum_gradient_bits"]])[0], f64([case["sum_hessian_bits"]])[0],
            case["num_data"])
        if not (_cand_equal(rev, case["cand_rev_bits"]) and _cand_equal(fwd, case["cand_fwd_bits"])):
            bad += 1
    assert bad >= 4


# --- xorshift64 (gradient_discretizer.rs:255-263): full period over GF(2) ---------
def _gf2_mul(a, b):
    """Columns of a @ b, with 64x64 GF(2) matrices stored as 64 column bit masks."""
    out = []
    for col in b:
        v, i = 0, 0
        while col:
            if col & 1:
                v ^= a[i]
            col >>= 1
            i += 1
        out.append(v)
    return out


def _gf2_pow(m, e):
    r = [1 << i for i in range(64)]
    while e:
        if e & 1:
            r = _gf2_mul(r, m)
        m = _gf2_mul(m, m)
        e >>= 1
    return r


def test_xorshift_transition_has_full_period():
    """The oracle's one-step map, read column by column from its raw states, is a
    GF(2) matrix T with T^(2^64-1) = I and T^((2^64-1)/p) != I for every prime p of
    2^64-1: the stream visits every nonzero state (a full-period xorshift triple).
    A wrong shift amount or direction gives a matrix that fails this."""
    T = [int(oracle.xorshift_states(1 << i, 1)[0]) for i in range(64)]
    eye = [1 << i for i in range(64)]
    order = (1 << 64) - 1
    assert _gf2_pow(T, order) == eye
    for p in (3, 5, 17, 257, 641, 65537, 6700417):
        assert order % p == 0
        assert _gf2_pow(T, order // p) != eye, p
    # linearity: the map of a sum of basis states is the xor of their images
    x = 0x9E3779B97F4A7C15 ^ 42
    img = 0
    for i in range(64):
        if (x >> i) & 1:
            img ^= T[i]
    assert int(oracle.xorshift_states(x, 1)[0]) == img
    # next_u01 is the top 53 bits of the state after the step
    st = oracle.xorshift_states(x, 5)
    u = oracle.xorshift_u01(x, 5)
    assert np.array_equal(u, (st >> np.uint64(11)).astype(np.float64) / 2.0 ** 53)


def test_xorshift_matches_the_published_13_7_17_stream():
    """Known answer for the shift triple itself: Marsaglia's xor64 generator
    ("Xorshift RNGs", J. Stat. Softw. 8(14), 2003: x ^= x << 13; x ^= x >> 7;
    x ^= x << 17) from its example seed 88172645463325252 emits 8748534153485358512,
    3040900993826735515, 3453997556048239312.  The full-period check above cannot tell
    (13, 7, 17) from its mirror (17, 7, 13), which is also full period; this does."""
    st = oracle.xorshift_states(88172645463325252, 3)
    assert [int(v) for v in st] == [8748534153485358512, 3040900993826735515,
                                     3453997556048239312]
    mirror = 88172645463325252
    m = (1 << 64) - 1
    mirror ^= (mirror << 17) & m
    mirror ^= mirror >> 7
    mirror ^= (mirror << 13) & m
    assert mirror != int(st[0])


def test_xorshift_period_check_has_teeth():
    """The same period check rejects a transition with one shift direction flipped."""
    def step(x):
        x ^= (x << 13) & ((1 << 64) - 1)
        x ^= (x << 7) & ((1 << 64) - 1)  # planted: left instead of right
        x ^= (x << 17) & ((1 << 64) - 1)
        return x
    T = [step(1 << i) for i in range(64)]
    assert _gf2_pow(T, (1 << 64) - 1) != [1 << i for i in range(64)]


# --- path_smooth_parity.rs:274-345 (the real binary, 13 gain-option cells) -------
def _path_smooth_inputs():
    from lightgbm_rs_amd import feature_mappers, feature_meta
    z = np.load(os.path.join(GOLD, "path_smooth.npz"))
    X, y = z["X"], z["y"].astype(np.float32)
    ms = feature_mappers(X, max_bin=63, min_data_in_leaf=5)
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    return z, X, y, bins, meta, ub


def path_smooth_cells():
    z = np.load(os.path.join(GOLD, "path_smooth.npz"))
    out, off = [], 0
    for i, (ps, mds, l1, nl) in enumerate(z["cells"]):
        counts = z["leaf_counts"][i]
        leaves = []
        for c in counts:
            leaves.append(z["leaf_flat"][off:off + c])
            off += c
        out.append(dict(ps=float(ps), mds=float(mds), l1=float(l1), nl=int(nl), leaves=leaves,
                        pred=z["pred_bits"][i].view(np.float64)))
    return out


@pytest.mark.parametrize("cell", range(13))
def test_path_smooth_cells_match_real_binary(cell):
    """Binary boosting with f32 gradients under every (path_smooth, max_delta_step,
    lambda_l1, num_leaves) cell: every tree's leaf values and the raw predictions.
    The reference gates these goldens at ORACLE_TOL = 1e-6 as f32; the oracle
    reproduces the real binary's f64 bits, so the test asserts bits."""
    z, X, y, bins, meta, ub = _path_smooth_inputs()
    c = path_smooth_cells()[cell]
    cfg = GainConfig.make(min_data_in_leaf=5, lambda_l1=c["l1"], max_delta_step=c["mds"],
                          path_smooth=c["ps"])
    iters = int(z["num_iterations"])
    scores, trees = oracle.train_binary(bins, meta, ub, y, cfg, c["nl"], -1, iters, 0.1,
                                        boost_from_average=True, quantized=False)
    assert len(trees) == iters
    for t, gold in zip(trees, c["leaves"]):
        lv = t["leaf_value"][:t["num_leaves"]]
        assert len(lv) == len(gold)
        assert np.array_equal(lv.view(np.uint64), np.ascontiguousarray(gold).view(np.uint64))
    assert np.array_equal(scores.view(np.uint64), np.ascontiguousarray(c["pred"]).view(np.uint64))


def test_path_smooth_cells_have_teeth():
    """Every cell whose option bites differs from the all-defaults control by more
    than the tolerance (path_smooth_parity.rs:350-398), so the cell tests above
    cannot pass on a learner that ignored the options."""
    cells = path_smooth_cells()
    ctrl = [c for c in cells if c["ps"] == 0 and c["mds"] == 0 and c["l1"] == 0][0]
    for c in cells:
        if c is ctrl or c["mds"] == 1e3 or c["nl"] != ctrl["nl"]:
            continue
        assert np.abs(c["pred"] - ctrl["pred"]).max() > 1e-6, (c["ps"], c["mds"], c["l1"])
