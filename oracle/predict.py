"""CPU restatement of the reference's model-text loader and batch predictor.

Test infrastructure only (the parity checker of the device predictor).  Follows
crates/lgbm-model/src/:
  model_text.rs:48-160  header keys (num_class, num_tree_per_iteration,
                        max_feature_idx, objective) and the Tree= blocks
  tree.rs:846-1000      Tree::parse (per-tree key=value fields)
  tree.rs:160-340       NumericalDecision / CategoricalDecision / GetLeaf
  tree.rs:279-316       linear leaves (leaf_const + sum coeff * x, NaN -> leaf_value)
  tree.rs:336-583       ExpectedValue and TreeSHAP (feature contributions),
                        predict.rs:607-697 their per-class layout
  ensemble.rs:75-102    init_predict + predict_raw (f64 accumulation per class,
                        iteration order)
  objective.rs:125-340  objective= parsing and ConvertOutput
  predict.rs:75-131     dense f32 rows widened to f64
Pinned by the reference's prediction goldens (tests/golden/predict/).
"""
import math

import numpy as np

K_ZERO_THRESHOLD = 1e-35
MISSING_NONE, MISSING_ZERO, MISSING_NAN = 0, 1, 2
CATEGORICAL_MASK, DEFAULT_LEFT_MASK = 1, 2


def _f64_list(v):
    return np.array([float(t) for t in v.split()], dtype=np.float64)


def _i_list(v, dtype=np.int64):
    return np.array([int(t) for t in v.split()], dtype=dtype)


def parse_tree(lines):
    kv = {}
    for line in lines:
        if not line:
            break
        k, _, v = line.partition("=")
        kv[k] = v
    t = {"num_leaves": int(kv["num_leaves"]), "num_cat": int(kv["num_cat"]),
         "leaf_value": _f64_list(kv["leaf_value"])}
    if t["num_leaves"] > 1:
        t["split_feature"] = _i_list(kv["split_feature"])
        t["threshold"] = _f64_list(kv["threshold"])
        t["decision_type"] = _i_list(kv["decision_type"])
        t["left_child"] = _i_list(kv["left_child"])
        t["right_child"] = _i_list(kv["right_child"])
        if t["num_cat"] > 0:
            t["cat_boundaries"] = _i_list(kv["cat_boundaries"])
            t["cat_threshold"] = _i_list(kv["cat_threshold"], np.uint64)
    # data counts (TreeSHAP covers); the reference's parser defaults them to 0
    t["leaf_count"] = _i_list(kv.get("leaf_count", " ".join(["0"] * t["num_leaves"])))
    if t["num_leaves"] > 1:
        t["internal_count"] = _i_list(kv.get("internal_count",
                                             " ".join(["0"] * (t["num_leaves"] - 1))))
    if int(kv.get("is_linear", "0")) != 0:
        # parse_linear_model (tree.rs:1341-1412): per-leaf groups of the flat streams
        const, counts = _f64_list(kv["leaf_const"]), _i_list(kv["num_features"])
        feats = _i_list(kv.get("leaf_features", ""))
        coeff = _f64_list(kv.get("leaf_coeff", ""))
        if len(const) != t["num_leaves"] or len(counts) != t["num_leaves"]:
            raise ValueError("linear leaf arrays != num_leaves")
        if (counts < 0).any() or len(feats) != counts.sum() or len(coeff) != counts.sum():
            raise ValueError("leaf_features / leaf_coeff length != sum(num_features)")
        off = np.concatenate([[0], np.cumsum(counts)])
        t["linear"] = [(const[l], feats[off[l]:off[l + 1]], coeff[off[l]:off[l + 1]])
                       for l in range(t["num_leaves"])]
    return t


def tree_output(t, X64):
    """Tree::predict (tree.rs:279-316): the leaf's value; for a linear tree the leaf's
    `leaf_const + sum coeff * x[feature]` added term by term, or the leaf's value when
    any of those features is NaN."""
    leaf = leaf_of(t, X64)
    out = t["leaf_value"][leaf]
    if "linear" not in t:
        return out
    out = out.copy()
    for l, (c, feats, coeff) in enumerate(t["linear"]):
        rows = np.nonzero(leaf == l)[0]
        v = np.full(len(rows), c)
        nan = np.zeros(len(rows), dtype=bool)
        for f, w in zip(feats, coeff):
            xv = X64[rows, f]
            nan |= np.isnan(xv)
            v = v + w * xv
        out[rows] = np.where(nan, t["leaf_value"][l], v)
    return out


def parse_model(text):
    lines = text.replace("\r", "").split("\n")
    head, head_lines, i = {}, set(), 0
    while i < len(lines) and not lines[i].startswith("Tree="):
        head_lines.add(lines[i])
        k, sep, v = lines[i].partition("=")
        if sep:
            head[k] = v
        i += 1
    trees = []
    while i < len(lines):
        if lines[i].startswith("Tree="):
            j = i + 1
            block = []
            while j < len(lines) and lines[j]:
                block.append(lines[j])
                j += 1
            trees.append(parse_tree(block))
            i = j
        elif lines[i].startswith("end of trees"):
            break
        else:
            i += 1
    num_class = int(head["num_class"])
    obj = head.get("objective", "").split() or [None]
    params = dict(t.split(":", 1) for t in obj[1:] if ":" in t)
    return {"num_class": num_class,
            "num_tree_per_iteration": int(head.get("num_tree_per_iteration", num_class)),
            "max_feature_idx": int(head["max_feature_idx"]),
            "objective": obj[0], "sqrt": "sqrt" in obj[1:],
            "sigmoid": float(params.get("sigmoid", "1")), "trees": trees,
            "average_output": "average_output" in head_lines}


def _decide(t, node, fval):
    """Next node for the rows at internal `node` (arrays), tree.rs:193-245."""
    dt = t["decision_type"][node]
    thr = t["threshold"][node]
    left, right = t["left_child"][node], t["right_child"][node]
    out = np.empty_like(node)
    cat = (dt & CATEGORICAL_MASK) > 0
    # numerical
    mt = (dt >> 2) & 3
    nan = np.isnan(fval)
    fv = np.where(nan & (mt != MISSING_NAN), 0.0, fval)
    is_zero = (fv >= -K_ZERO_THRESHOLD) & (fv <= K_ZERO_THRESHOLD)
    missing = ((mt == MISSING_ZERO) & is_zero) | ((mt == MISSING_NAN) & np.isnan(fv))
    dleft = (dt & DEFAULT_LEFT_MASK) > 0
    num_next = np.where(missing, np.where(dleft, left, right), np.where(fv <= thr, left, right))
    out[:] = num_next
    if cat.any():
        idx = np.nonzero(cat)[0]
        for r in idx:  # categorical rows: small cases only
            v = fval[r]
            if math.isnan(v):
                out[r] = right[r]
                continue
            iv = int(v) if abs(v) < 2 ** 31 else (2 ** 31 - 1 if v > 0 else -2 ** 31)
            if iv < 0:
                out[r] = right[r]
                continue
            ci = int(thr[r])
            lo, hi = t["cat_boundaries"][ci], t["cat_boundaries"][ci + 1]
            w = iv // 32
            hit = w < hi - lo and (int(t["cat_threshold"][lo + w]) >> (iv % 32)) & 1
            out[r] = left[r] if hit else right[r]
    return out


def leaf_of(t, X64):
    n = X64.shape[0]
    if t["num_leaves"] <= 1:
        return np.zeros(n, dtype=np.int64)
    node = np.zeros(n, dtype=np.int64)
    rows = np.arange(n)
    active = node >= 0
    while active.any():
        r = rows[active]
        nd = node[r]
        fval = X64[r, t["split_feature"][nd]]
        node[r] = _decide(t, nd, fval)
        active = node >= 0
    return ~node


def _range(model, start_iteration, num_iteration):
    ntpi = model["num_tree_per_iteration"]
    total = len(model["trees"]) // ntpi
    start = min(max(start_iteration, 0), total)
    num = min(num_iteration, total - start) if num_iteration > 0 else total - start
    return start, num


def predict(model, X, start_iteration=0, num_iteration=-1, kind="raw"):
    """kind: 'raw' (f64 [rows, ntpi]), 'transformed', or 'leaf' (int [rows, trees])."""
    X64 = np.asarray(X, dtype=np.float32).astype(np.float64)
    ntpi = model["num_tree_per_iteration"]
    start, num = _range(model, start_iteration, num_iteration)
    trees = model["trees"]
    if kind == "leaf":
        cols = [leaf_of(trees[i * ntpi + k], X64) for i in range(start, start + num)
                for k in range(ntpi)]
        return np.stack(cols, axis=1) if cols else np.zeros((X64.shape[0], 0), np.int64)
    raw = np.zeros((X64.shape[0], ntpi), dtype=np.float64)
    for i in range(start, start + num):
        for k in range(ntpi):
            t = trees[i * ntpi + k]
            raw[:, k] = raw[:, k] + tree_output(t, X64)
    if kind == "raw":
        return raw
    if model["objective"] is None:
        raise ValueError("model has no objective= line; cannot apply ConvertOutput")
    if model["average_output"] and num > 0:
        # predict.rs:338-349: RF divides the raw sum by the iteration count first
        raw = raw / float(num)
    return convert(model, raw)


def convert(model, raw):
    obj, out = model["objective"], np.empty_like(raw)
    sig = model["sigmoid"]
    for r in range(raw.shape[0]):
        v = raw[r]
        if obj in ("binary",):
            out[r, 0] = 1.0 / (1.0 + math.exp(-sig * v[0]))
        elif obj in ("cross_entropy", "xentropy"):
            out[r, 0] = 1.0 / (1.0 + math.exp(-v[0]))
        elif obj in ("cross_entropy_lambda", "xentlambda"):
            out[r, 0] = math.log1p(math.exp(v[0]))
        elif obj in ("poisson", "gamma", "tweedie"):
            out[r, 0] = math.exp(v[0])
        elif obj in ("multiclass", "softmax"):
            wmax = v[0]
            for x in v[1:]:
                wmax = max(x, wmax)
            e = [math.exp(x - wmax) for x in v]
            s = 0.0
            for x in e:
                s += x
            out[r] = [x / s for x in e]
        elif obj in ("multiclassova", "multiclass_ova", "ova", "ovr"):
            out[r] = [1.0 / (1.0 + math.exp(-sig * x)) for x in v]
        else:  # regression family
            x = v[0]
            out[r, 0] = (math.copysign(1.0, x) if x != 0 else 0.0) * x * x if model["sqrt"] else x
    return out


def _es_stop(out, margin):
    """pred_early_stop_should_stop (crates/lgbm-model/src/ensemble.rs:337-356)."""
    if len(out) == 1:
        return 2.0 * abs(out[0]) > margin
    top1 = top2 = -math.inf
    for v in out:
        if v > top1:
            top2, top1 = top1, v
        elif v > top2:
            top2 = v
    return (top1 - top2) > margin


def predict_early_stop(model, X, freq, margin, start_iteration=0, num_iteration=-1):
    """GbdtModel::predict_raw_early_stop per row (ensemble.rs:120-151) behind the
    accurate-prediction gate of predict_raw_early_stop_mat (predict.rs:557-605):
    returns (raw [rows, ntpi] float64, iterations evaluated [rows])."""
    if model["objective"] not in ("binary", "multiclass", "softmax", "multiclassova",
                                  "multiclass_ova", "ova", "ovr"):
        freq = 0
    X64 = np.asarray(X, dtype=np.float32).astype(np.float64)
    ntpi = model["num_tree_per_iteration"]
    start, num = _range(model, start_iteration, num_iteration)
    trees = model["trees"]
    vals = [[tree_output(trees[i * ntpi + k], X64) for k in range(ntpi)]
            for i in range(start, start + num)]
    raw = np.zeros((len(X64), ntpi))
    iters = np.zeros(len(X64), np.int32)
    for r in range(len(X64)):
        out = [0.0] * ntpi
        counter = 0
        n = 0
        for ii in range(num):
            for k in range(ntpi):
                out[k] += vals[ii][k][r]
            n += 1
            counter += 1
            if freq > 0 and counter == freq:
                if _es_stop(out, margin):
                    break
                counter = 0
        raw[r] = out
        iters[r] = n
    return raw, iters


# ---- TreeSHAP (feature contributions) ---------------------------------------------
# Lundberg et al., "Consistent Individualized Feature Attribution for Tree Ensembles"
# (arXiv:1706.06060), Algorithm 2, in the form the reference uses (tree.rs:336-583):
# covers are the data counts, each recursion frame copies its parent's unique path
# forward in one flat buffer, and every product / quotient keeps the association the
# reference writes, so the f64 results agree bit for bit.

def _count(t, node):
    return float(t["internal_count"][node]) if node >= 0 else float(t["leaf_count"][~node])


def expected_value(t):
    """Tree::expected_value (tree.rs:351-361): the cover-weighted leaf average."""
    if t["num_leaves"] == 1:
        return float(t["leaf_value"][0])
    total = float(t["internal_count"][0])
    e = 0.0
    for i in range(t["num_leaves"]):
        e += (float(t["leaf_count"][i]) / total) * float(t["leaf_value"][i])
    return e


def _extend(path, b, d, zf, of, feat):
    """ExtendPath (tree.rs:413-433) on the frame starting at path[b]."""
    path[b + d] = [feat, zf, of, 1.0 if d == 0 else 0.0]
    for i in range(d - 1, -1, -1):
        prev = path[b + i][3]
        path[b + i + 1][3] += of * prev * (i + 1.0) / (d + 1.0)
        path[b + i][3] = zf * prev * (d - i) / (d + 1.0)


def _unwind(path, b, d, k):
    """UnwindPath (tree.rs:435-460)."""
    of, zf = path[b + k][2], path[b + k][1]
    nxt = path[b + d][3]
    for i in range(d - 1, -1, -1):
        if of != 0.0:
            tmp = path[b + i][3]
            path[b + i][3] = nxt * (d + 1.0) / ((i + 1.0) * of)
            nxt = tmp - path[b + i][3] * zf * (d - i) / (d + 1.0)
        else:
            path[b + i][3] = (path[b + i][3] * (d + 1.0)) / (zf * (d - i))
    for i in range(k, d):
        path[b + i][0:3] = path[b + i + 1][0:3]


def _unwound_sum(path, b, d, k):
    """UnwoundPathSum (tree.rs:462-485)."""
    of, zf = path[b + k][2], path[b + k][1]
    nxt = path[b + d][3]
    total = 0.0
    for i in range(d - 1, -1, -1):
        if of != 0.0:
            tmp = nxt * (d + 1.0) / ((i + 1.0) * of)
            total += tmp
            nxt = path[b + i][3] - tmp * zf * ((d - i) / (d + 1.0))
        else:
            total += (path[b + i][3] / zf) / ((d - i) / (d + 1.0))
    return total


def _shap(t, x, phi, node, d, path, b, pz, po, pf):
    """TreeSHAP (tree.rs:487-583); the frame of this call starts at path[b + d]."""
    for i in range(d):
        path[b + d + i] = list(path[b + i])
    b += d
    _extend(path, b, d, pz, po, pf)
    if node < 0:
        lv = float(t["leaf_value"][~node])
        for i in range(1, d + 1):
            w = _unwound_sum(path, b, d, i)
            el = path[b + i]
            phi[el[0]] += w * (el[2] - el[1]) * lv
        return
    f = int(t["split_feature"][node])
    hot = int(_decide(t, np.array([node]), np.array([x[f]], dtype=np.float64))[0])
    cold = int(t["right_child"][node]) if hot == t["left_child"][node] else int(t["left_child"][node])
    w = _count(t, node)
    hz, cz = _count(t, hot) / w, _count(t, cold) / w
    iz, io = 1.0, 1.0
    k = 0
    while k <= d and path[b + k][0] != f:
        k += 1
    nd = d
    if k != d + 1:
        iz, io = path[b + k][1], path[b + k][2]
        _unwind(path, b, d, k)
        nd -= 1
    _shap(t, x, phi, hot, nd + 1, path, b, hz * iz, io, f)
    _shap(t, x, phi, cold, nd + 1, path, b, cz * iz, 0.0, f)


def _max_depth(t):
    if t["num_leaves"] <= 1:
        return 0
    best, stack = 0, [(0, 0)]
    while stack:
        n, dep = stack.pop()
        if n < 0:
            best = max(best, dep)
        else:
            stack += [(int(t["left_child"][n]), dep + 1), (int(t["right_child"][n]), dep + 1)]
    return best


def predict_contrib(model, X, start_iteration=0, num_iteration=-1):
    """predict_contrib_mat (predict.rs:607-697): per row and class a block of
    max_feature_idx + 1 feature contributions and the expected-value base, summed over
    the iterations in order (f32 rows widened to f64).  Pure Python: small inputs."""
    if any("linear" in t for t in model["trees"]):
        raise ValueError("feature contributions are not defined for linear trees")
    X64 = np.asarray(X, dtype=np.float32).astype(np.float64)
    ntpi, nf = model["num_tree_per_iteration"], model["max_feature_idx"] + 1
    start, num = _range(model, start_iteration, num_iteration)
    out = np.zeros((X64.shape[0], ntpi * (nf + 1)))
    for r in range(X64.shape[0]):
        row = out[r]
        for i in range(start, start + num):
            for k in range(ntpi):
                t = model["trees"][i * ntpi + k]
                phi = row[k * (nf + 1):(k + 1) * (nf + 1)]
                phi[nf] += expected_value(t)
                if t["num_leaves"] > 1:
                    L = _max_depth(t) + 1
                    path = [[0, 0.0, 0.0, 0.0] for _ in range(L * (L + 1) // 2)]
                    _shap(t, X64[r], phi, 0, 0, path, 0, 1.0, 1.0, -1)
    return out
