"""Extract the reference's committed golden vectors into compact JSON fixtures.

Run in the build container (where /root/reference exists):

    python tests/golden/make_golden.py

The reference's fixtures are data (inputs + expected outputs as raw IEEE bit
patterns); this script only re-encodes them.  Sources (under
/root/reference/crates/oracle-harness/tests/fixtures/):

  kernels/histogram.txt   -> hist_f64.json      (format: kernel_parity.rs:17-25)
  kernels/split.txt       -> split_scan.json    (format: kernel_parity.rs:285-360)
  kernels/subtract.txt    -> subtract.json
  kernels/partition.txt   -> partition.json     (format: kernel_parity.rs:1162-1220)
  learner/spine_real.txt, learner/mfb_pos_real.txt, na_missing/model_real.txt,
  gain_params/{penalty,max_delta_step,path_smooth}/model_real.txt,
  categorical/{cat_onehot,cat_manyvsmany}.{txt,bins.json} -> learner_real.json
      (real lib_lightgbm 4.6 model text; the corpora are the ones the reference
       tests drive: learner_parity.rs:1214-1330 and 1455-1483,
       na_missing_parity.rs:108-141, gain_params_parity.rs:93-226)
  boosting/multiclass_{scores,gh_iter1,gh_iterN}.txt, multiclass_spine_model.txt
      -> multiclass_spine.json (boosting_parity.rs:110-170, 1259-1300)
  path_smooth/path_smooth_golden.json -> path_smooth.npz
      (real lightgbm 4.6 boosting runs; path_smooth_parity.rs:226-345)

plus the hand-computed discretizer cases of
crates/lgbm-treelearner/src/gradient_discretizer.rs:269-333 -> discretizer_cases.json.
"""
import json
import os
import struct
import sys

REF = "/root/reference/crates/oracle-harness/tests/fixtures"
OUT = os.path.dirname(os.path.abspath(__file__))


def field(tokens, key):
    for t in tokens:
        if t.startswith(key + "="):
            return t[len(key) + 1:]
    return None


def ints(s):
    return [int(x) for x in s.split(";")] if s else []


def read(path):
    with open(os.path.join(REF, path)) as f:
        return [ln.rstrip("\n") for ln in f]


def hist_cases():
    lines = [l for l in read("kernels/histogram.txt") if l and not l.startswith("#")]
    out, i = [], 0
    while i < len(lines):
        t = lines[i].split()
        if t[0] != "HCASE":
            i += 1
            continue
        name = field(t, "name")
        num_bin = int(field(t, "num_bin"))
        bins = ints(lines[i + 1].split()[1] if len(lines[i + 1].split()) > 1 else "")
        grad = ints(lines[i + 2].split()[1] if len(lines[i + 2].split()) > 1 else "")
        hess = ints(lines[i + 3].split()[1] if len(lines[i + 3].split()) > 1 else "")
        hist = ints(lines[i + 4].split()[1])
        assert lines[i + 1].startswith("BINS") and lines[i + 4].startswith("HIST")
        nz = [[k, v] for k, v in enumerate(hist) if v != 0]
        out.append(dict(name=name, num_bin=num_bin, bins=bins, grad_bits=grad, hess_bits=hess,
                        hist_len=len(hist), hist_nonzero_bits=nz))
        i += 5
    return out


def split_cases():
    lines = [l for l in read("kernels/split.txt") if l and not l.startswith("#")]
    out, i = [], 0
    keys_i = ["num_bin", "offset", "default_bin", "skip_default_bin", "na_as_missing", "use_l1",
              "min_data_in_leaf", "num_data"]
    keys_f = ["min_sum_hessian_in_leaf", "lambda_l1", "lambda_l2", "min_gain_to_split",
              "sum_gradient", "sum_hessian"]
    while i < len(lines):
        t = lines[i].split()
        if t[0] != "SCASE":
            i += 1
            continue
        c = dict(name=field(t, "name"))
        for k in keys_i:
            c[k] = int(field(t, k))
        for k in keys_f:
            c[k + "_bits"] = int(field(t, k))
        c["hist_bits"] = ints(lines[i + 1].split()[1])
        c["cand_rev_bits"] = ints(lines[i + 2].split()[1]) if len(lines[i + 2].split()) > 1 else []
        c["cand_fwd_bits"] = ints(lines[i + 3].split()[1]) if len(lines[i + 3].split()) > 1 else []
        w = lines[i + 4].split()
        assert w[0] == "SWIN"
        win = {}
        for k in ["is_splittable", "threshold", "left_count", "right_count", "default_left"]:
            win[k] = int(field(w, k))
        for k in ["gain", "min_gain_shift", "left_sum_gradient", "left_sum_hessian",
                  "right_sum_gradient", "right_sum_hessian", "left_output", "right_output"]:
            win[k + "_bits"] = int(field(w, k))
        c["win"] = win
        out.append(c)
        i += 5
    return out


def subtract_cases():
    lines = [l for l in read("kernels/subtract.txt") if l and not l.startswith("#")]
    out, i = [], 0
    while i < len(lines):
        t = lines[i].split()
        if t[0] != "SUBCASE":
            i += 1
            continue
        out.append(dict(name=field(t, "name"), parent_bits=ints(lines[i + 1].split()[1]),
                        child_bits=ints(lines[i + 2].split()[1]),
                        derived_bits=ints(lines[i + 3].split()[1])))
        i += 4
    return out


def partition_cases():
    lines = [l for l in read("kernels/partition.txt") if l and not l.startswith("#")]
    out, i = [], 0
    while i < len(lines):
        t = lines[i].split()
        if t[0] != "PCASE":
            i += 1
            continue
        c = dict(name=field(t, "name"))
        for k in ["num_bin", "min_bin", "max_bin", "threshold", "most_freq_bin", "missing_type",
                  "default_bin", "default_left"]:
            c[k] = int(field(t, k))
        c["bins"] = ints(lines[i + 1].split()[1])
        c["order"] = ints(lines[i + 2].split()[1])
        c["split_point"] = int(lines[i + 3].split()[1])
        out.append(c)
        i += 4
    return out


def parse_model_tree(path):
    """Tree=0 block of a LightGBM v4 model text -> dict of string lists."""
    tree, inside = {}, False
    for ln in read(path):
        if ln.startswith("Tree=0"):
            inside = True
            continue
        if inside:
            if not ln.strip():
                break
            k, _, v = ln.partition("=")
            tree[k] = v.split()
    return tree


def parse_model_trees(path):
    """Every Tree=i block of a LightGBM v4 model text -> list of dicts of string lists."""
    trees, cur = [], None
    for ln in read(path):
        if ln.startswith("Tree="):
            cur = {}
            trees.append(cur)
            continue
        if cur is not None:
            if not ln.strip():
                cur = None
                continue
            k, _, v = ln.partition("=")
            cur[k] = v.split()
    return trees


def multiclass_spine():
    """boosting/multiclass_* (the real lightgbm 4.6 binary; boosting_parity.rs:110-170,
    1259-1300): the 12-row, 2-feature, 3-class corpus, 5 iterations, lr 0.1,
    num_leaves 4, min_data_in_leaf 1, boost_from_average; the per-iteration
    class-major raw scores (f64 bits), the iteration-1 and iteration-4 gradients
    (f32 bits) and the 15 trees of the model text."""
    f0 = [0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5]
    f1 = [0, 1, 2, 0, 1, 2, 0, 1, 2, 0, 1, 2]
    labels = [0.0, 0.0, 0.0, 1.0, 1.0, 1.0, 2.0, 2.0, 2.0, 0.0, 1.0, 2.0]
    scores = [[int(t) for t in ln.split()] for ln in read("boosting/multiclass_scores.txt")
              if ln.strip() and not ln.startswith("#")]

    def gh(name):
        out = {}
        for ln in read(name):
            if ln.startswith("GRAD") or ln.startswith("HESS"):
                k, *v = ln.split()
                out[k] = [int(t) for t in v]
        return out
    trees = parse_model_trees("boosting/multiclass_spine_model.txt")
    keep = ("num_leaves", "split_feature", "threshold", "decision_type", "left_child",
            "right_child", "leaf_value", "leaf_count", "internal_count")
    return dict(X=[[a, b] for a, b in zip(f0, f1)], labels=labels, num_class=3,
                num_iterations=5, learning_rate=0.1, num_leaves=4, min_data_in_leaf=1,
                score_bits=scores, gh_iter1=gh("boosting/multiclass_gh_iter1.txt"),
                gh_iter4=gh("boosting/multiclass_gh_iterN.txt"),
                trees=[{k: t[k] for k in keep if k in t} for t in trees])


def f64bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def real_upper_bounds(num_bin, zero_sentinel_bin0=False):
    # learner_parity.rs:1070-1085 / 1112-1118: midpoint (b + 0.5) + 1 ULP; the mfb>0
    # corpus carries kZeroThreshold = 1e-35f widened at bin 0.
    out = []
    for b in range(num_bin):
        out.append(struct.unpack("<d", struct.pack("<Q", f64bits(b + 0.5) + 1))[0])
    if zero_sentinel_bin0:
        out[0] = struct.unpack("<f", struct.pack("<f", 1e-35))[0]
    return out


def learner_real():
    cases = []
    # learner_parity.rs:1214-1230 (spine_real)
    cases.append(dict(
        name="spine_real", golden_file="learner/spine_real.txt",
        bins=[0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5],
        grad=[-6.0, -6.0, -5.0, -5.0, -1.0, -1.0, 1.0, 1.0, 5.0, 5.0, 6.0, 6.0],
        num_bin=6, most_freq_bin=0, upper=real_upper_bounds(6),
        tree=parse_model_tree("learner/spine_real.txt")))
    # learner_parity.rs:1297-1330 (mfb_pos_real)
    cases.append(dict(
        name="mfb_pos_real", golden_file="learner/mfb_pos_real.txt",
        bins=[0, 1, 2, 2, 2, 2, 2, 2, 3, 3, 1, 0],
        grad=[-6.0, -3.0, -1.0, -1.0, -1.0, 1.0, 1.0, 1.0, 4.0, 5.0, -3.0, -6.0],
        num_bin=4, most_freq_bin=0, upper=real_upper_bounds(4, zero_sentinel_bin0=True),
        tree=parse_model_tree("learner/mfb_pos_real.txt")))
    for c in cases:
        # single_feature_corpus (learner_parity.rs:1039-1062)
        c.update(hess=[1.0] * len(c["grad"]), min_data_in_leaf=1, min_sum_hessian_in_leaf=1e-3,
                 num_leaves=4, max_depth=-1, shrinkage=0.1)
    # na_missing_parity.rs:108-141: NaN rows carry the top bin (num_bin - 1), missing
    # type NaN, offset 1, default_bin out of range; num_leaves 2
    cases.append(dict(
        name="na_missing_real", golden_file="na_missing/model_real.txt",
        bins=[0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5],
        grad=[-6.0, -6.0, -5.0, -5.0, -1.0, -1.0, 1.0, 1.0, 5.0, 5.0, 6.0, 6.0],
        num_bin=6, most_freq_bin=0, missing_type=2, default_bin=6,
        upper=real_upper_bounds(6), tree=parse_model_tree("na_missing/model_real.txt"),
        hess=[1.0] * 12, min_data_in_leaf=1, min_sum_hessian_in_leaf=1e-3, num_leaves=2,
        max_depth=-1, shrinkage=0.1))
    # gain_params_parity.rs:93-226: one corpus, three gain options (feature_contri 0.5,
    # max_delta_step 0.7, path_smooth 2.0); split_gain compared too
    for which, extra in (("penalty", dict(feature_contri=[0.5])),
                         ("max_delta_step", dict(max_delta_step=0.7)),
                         ("path_smooth", dict(path_smooth=2.0))):
        c = dict(name="gain_params_" + which, golden_file=f"gain_params/{which}/model_real.txt",
                 bins=[0, 0, 1, 1, 2, 2, 3, 3, 4, 4],
                 grad=[-6.0, -6.0, -5.0, -5.0, -1.0, -1.0, 1.0, 1.0, 6.0, 6.0],
                 num_bin=5, most_freq_bin=0, missing_type=0, default_bin=5,
                 upper=real_upper_bounds(5),
                 tree=parse_model_tree(f"gain_params/{which}/model_real.txt"),
                 hess=[1.0] * 10, min_data_in_leaf=1, min_sum_hessian_in_leaf=1e-3,
                 num_leaves=2, max_depth=-1, shrinkage=0.1, check_split_gain=True)
        c.update(extra)
        cases.append(c)
    # learner_parity.rs:1455-1483 (cat_corpus): one categorical feature, hess 1,
    # missing type None, default_bin = num_bin; the feature's per-bin values are its
    # bin -> category map (bin 0 is the NaN dummy, category -1)
    for name in ("cat_onehot", "cat_manyvsmany"):
        with open(os.path.join(REF, f"categorical/{name}.bins.json")) as f:
            s = json.load(f)
        n = len(s["grad"])
        cases.append(dict(
            name=name + "_real", golden_file=f"categorical/{name}.txt",
            bins=s["bins"], grad=s["grad"], num_bin=s["num_bin"],
            most_freq_bin=s["most_freq_bin"], missing_type=0, default_bin=s["num_bin"],
            bin_type=1, upper=[float(v) for v in s["bin_2_categorical"]],
            tree=parse_model_tree(f"categorical/{name}.txt"), hess=[1.0] * n,
            min_data_in_leaf=1, min_sum_hessian_in_leaf=1e-3, num_leaves=s["num_leaves"],
            max_depth=-1, shrinkage=s["shrinkage"], check_split_gain=True,
            cat=dict(cat_l2=s["cat_l2"], cat_smooth=s["cat_smooth"],
                     min_data_per_group=s["min_data_per_group"],
                     max_cat_threshold=s["max_cat_threshold"],
                     max_cat_to_onehot=s["max_cat_to_onehot"])))
    for c in cases:
        c["upper_bits"] = [f64bits(x) for x in c.pop("upper")]
    return cases


def path_smooth_golden():
    """path_smooth/path_smooth_golden.json (the real lightgbm 4.6 binary, capture.py:
    800 x 10 N(0,1) features, binary labels, 8 iterations, max_bin 63,
    min_data_in_leaf 5, 13 (path_smooth, max_delta_step, lambda_l1, num_leaves) cells)
    -> path_smooth.npz: X [800, 10] f64, y, cells [13, 4], per-cell raw predictions
    and leaf values (flattened, with per-tree counts)."""
    import numpy as np
    with open(os.path.join(REF, "path_smooth/path_smooth_golden.json")) as f:
        d = json.load(f)
    n, m = d["num_rows"], d["num_cols"]
    X = np.array([int(h, 16) for h in d["features_bits"]], dtype=np.uint64).view(np.float64)
    y = np.array([int(h, 16) for h in d["labels_bits"]], dtype=np.uint64).view(np.float64)
    cells, preds, flat, counts = [], [], [], []
    for key in sorted(d["cells"]):
        c = d["cells"][key]
        cells.append([c["path_smooth"], c["max_delta_step"], c["lambda_l1"], c["num_leaves"]])
        preds.append(np.array([int(h, 16) for h in c["pred_bits"]], dtype=np.uint64))
        counts.append([len(t) for t in c["leaf_values"]])
        for t in c["leaf_values"]:
            flat.extend(t)
    out = os.path.join(OUT, "path_smooth.npz")
    np.savez_compressed(out, X=X.reshape(n, m), y=y, cells=np.array(cells, dtype=np.float64),
                        pred_bits=np.stack(preds), leaf_flat=np.array(flat, dtype=np.float64),
                        leaf_counts=np.array(counts, dtype=np.int32),
                        num_iterations=np.int32(d["num_iterations"]))
    return len(cells), out


def col_sampler_golden():
    """learner/col_sampler.txt (the genuine Random::Sample transcription driven as the
    learner drives it): one sampler, its per-tree selection, then five per-node
    draws in order."""
    out = {"nodes": []}
    for ln in read("learner/col_sampler.txt"):
        if ln.startswith("CS_CONFIG"):
            kv = dict(t.split("=") for t in ln.split()[1:])
            out["feature_fraction"] = struct.unpack("<d", struct.pack("<Q", int(kv["feature_fraction_bits"])))[0]
            out["feature_fraction_bynode"] = struct.unpack(
                "<d", struct.pack("<Q", int(kv["feature_fraction_bynode_bits"])))[0]
            out["seed"] = int(kv["seed"])
            out["num_features"] = int(kv["num_features"])
        elif ln.startswith("CS_BYTREE"):
            out["bytree"] = [int(t) for t in ln.split()[1].split(";")]
        elif ln.startswith("CS_NODE"):
            out["nodes"].append([int(t) for t in ln.split()[2].split(";")])
    return out


def feature_fraction_golden():
    """feature_fraction/feature_fraction_golden.json (the real lightgbm 4.6 binary,
    capture.py: 600 x 20 N(0,1), binary labels, 8 iterations, num_leaves 8,
    min_data_in_leaf 5, max_bin 63, feature_fraction_seed 2) -> feature_fraction.npz:
    the per-tree column sampling cells (feature_fraction_bynode = 1): raw predictions
    (f64 bits) and each tree's set of split features."""
    import numpy as np
    with open(os.path.join(REF, "feature_fraction/feature_fraction_golden.json")) as f:
        d = json.load(f)
    n, m = d["num_rows"], d["num_cols"]
    X = np.array([int(h, 16) for h in d["features_bits"]], dtype=np.uint64).view(np.float64)
    y = np.array([int(h, 16) for h in d["labels_bits"]], dtype=np.uint64).view(np.float64)
    fracs, preds, flat, counts = [], [], [], []
    for key in sorted(d["cells"]):
        c = d["cells"][key]
        if c["feature_fraction_bynode"] != 1.0:
            continue
        fracs.append(c["feature_fraction"])
        preds.append(np.array([int(h, 16) for h in c["pred_bits"]], dtype=np.uint64))
        counts.append([len(t) for t in c["per_tree_split_features"]])
        for t in c["per_tree_split_features"]:
            flat.extend(t)
    out = os.path.join(OUT, "feature_fraction.npz")
    np.savez_compressed(out, X=X.reshape(n, m), y=y, fractions=np.array(fracs, dtype=np.float64),
                        pred_bits=np.stack(preds), split_flat=np.array(flat, dtype=np.int32),
                        split_counts=np.array(counts, dtype=np.int32),
                        num_iterations=np.int32(d["num_iterations"]))
    return len(fracs), out


def lambdarank_golden():
    """rank/ (the real lightgbm 4.6 binary, xtask/py/rank_oracle_capture.py): the
    30-row, 6-query corpus (X: RandomState(20240607).randint(0, 8, (30, 3)), the
    recipe's first draw; labels from the scores golden), the iteration-1 gradients
    at zero scores (f32 bits; sigmoid 1, lambdarank_norm, truncation level 5), the
    final raw scores of the 10-iteration model (f64 bits) and its trees (num_leaves
    7, learning_rate 0.1, min_data_in_leaf 1, max_bin 255, min_data_in_bin 1)."""
    import numpy as np
    sc = {}
    for ln in read("rank/lambdarank_scores.txt"):
        if "=" in ln and not ln.startswith("#"):
            k, _, v = ln.partition("=")
            sc[k] = [int(t) for t in v.split(",")]
    gh = {}
    for ln in read("rank/lambdarank_gh_iter1.txt"):
        if ln.startswith("GRAD") or ln.startswith("HESS"):
            k, *v = ln.split()
            gh[k] = [int(t) for t in v]
    rng = np.random.RandomState(20240607)
    X = rng.randint(0, 8, size=(30, 3)).astype(np.float64)
    labels = rng.randint(0, 4, size=30).astype(np.float32)
    lab_bits = np.array(sc["labels"], dtype=np.uint32).view(np.float32)
    assert np.array_equal(labels, lab_bits), "the corpus recipe reproduces the golden labels"
    trees = parse_model_trees("rank/rank_lambdarank_byq0_es0_model.txt")
    keep = ("num_leaves", "split_feature", "threshold", "decision_type", "left_child",
            "right_child", "leaf_value", "leaf_count", "internal_count", "leaf_weight")
    return dict(X=X.tolist(), label_bits=sc["labels"], query_boundaries=sc["query_boundaries"],
                score_bits=sc["scores"], gh_iter1=gh, num_iterations=10, num_leaves=7,
                learning_rate=0.1, min_data_in_leaf=1, sigmoid=1.0, lambdarank_norm=True,
                truncation_level=5, trees=[{k: t[k] for k in keep if k in t} for t in trees])


def discretizer_cases():
    # Hand-computed unit cases, gradient_discretizer.rs:269-333 (inputs -> expected ints).
    return [
        dict(name="deterministic_quantize_constant_hessian_bins4", bins=4, const_hess=1,
             grad=[1.0, -1.0, 0.5, -0.5, 0.3, -0.3], hess=[1.0] * 6,
             grad_scale=0.5, q_grad=[2, -2, 1, -1, 1, -1], q_hess=[1] * 6),
        dict(name="half_rounds_away_from_zero", bins=4, const_hess=1,
             grad=[0.75, -0.75, 1.0], hess=[1.0] * 3, q_grad_sel={"0": 2, "1": -2}),
        dict(name="nonconstant_hessian_uses_full_bins", bins=4, const_hess=0,
             grad=[0.5, -0.5], hess=[0.25, 0.125], hess_scale=0.0625, q_hess=[4, 2]),
        dict(name="int_histogram_sums_per_bin", bins=4, const_hess=1,
             grad=[1.0, -1.0, 0.5, -0.5], hess=[1.0] * 4, binned=[0, 0, 1, 1], num_bin=2,
             int_hist=[0, 2, 0, 2]),
    ]


def main():
    if not os.path.isdir(REF):
        sys.exit("reference fixtures not found at " + REF)
    outs = {
        "hist_f64.json": hist_cases(),
        "split_scan.json": split_cases(),
        "subtract.json": subtract_cases(),
        "partition.json": partition_cases(),
        "learner_real.json": learner_real(),
        "discretizer_cases.json": discretizer_cases(),
        "multiclass_spine.json": multiclass_spine(),
        "col_sampler.json": col_sampler_golden(),
        "lambdarank.json": lambdarank_golden(),
    }
    for name, data in outs.items():
        with open(os.path.join(OUT, name), "w") as f:
            json.dump(data, f, separators=(",", ":"))
        print(name, len(data), os.path.getsize(os.path.join(OUT, name)), "bytes")
    for fn in (path_smooth_golden, feature_fraction_golden):
        k, path = fn()
        print(os.path.basename(path), k, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
