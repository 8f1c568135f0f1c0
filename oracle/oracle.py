"""ctypes wrapper of the CPU oracle (oracle/liblgbm_oracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The oracle restates the reference CPU learner
(see lgbm_oracle.cpp for the file:line map) and is the checker for the HIP path.
"""
import ctypes as C
import os
import subprocess

import numpy as np

from lightgbm_rs_amd._abi import (BatchedFeature, FeatureMeta, GainConfig, LayoutBuffers,
                                  SplitInfo, TreeBuffers, ptr)

def _cat_words(meta, upper, num_leaves):
    """cat_threshold capacity for a tree: (num_leaves - 1) x the widest category
    bitset of one node (largest non-negative category value / 32 + 1), at least the
    default 64 words a node."""
    per = 64
    if upper is not None:
        off = 0
        for m in meta:
            nb = int(m.num_bin)
            if int(m.bin_type) != 0:
                v = np.asarray(upper[off:off + nb], np.float64)
                v = v[(v >= 0) & (v < 2.0 ** 31)]
                if len(v):
                    per = max(per, int(v.max()) // 32 + 1)
            off += nb
    return max(num_leaves - 1, 1) * per


def _tree_buffers(num_leaves, meta, upper):
    return TreeBuffers(num_leaves, _cat_words(meta, upper, num_leaves))


_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblgbm_oracle.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.oracle_binary_boost_from_score.restype = C.c_double
        L.oracle_regression_boost_from_score.restype = C.c_double
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        buf = C.create_string_buffer(512)
        lib().oracle_last_error(buf, 512)
        raise RuntimeError(f"oracle error {rc}: {buf.value.decode()}")


def set_threads(n):
    return lib().oracle_set_threads(int(n))


def construct_histogram(bins, grad, hess, num_bin):
    bins = np.ascontiguousarray(bins, dtype=np.uint32)
    grad = np.ascontiguousarray(grad, dtype=np.float32)
    hess = np.ascontiguousarray(hess, dtype=np.float32)
    out = np.zeros(2 * num_bin, dtype=np.float64)
    _check(lib().oracle_construct_histogram(ptr(bins, C.c_uint32), ptr(grad, C.c_float),
                                            ptr(hess, C.c_float), C.c_int64(len(bins)),
                                            C.c_uint32(num_bin), ptr(out, C.c_double)))
    return out


def int_histogram(binned, disc, rows, num_bin):
    binned = np.ascontiguousarray(binned, dtype=np.uint32)
    disc = np.ascontiguousarray(disc, dtype=np.int8)
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    out = np.zeros(2 * num_bin, dtype=np.int64)
    _check(lib().oracle_construct_int_histogram(ptr(binned, C.c_uint32), ptr(disc, C.c_int8),
                                                ptr(rows, C.c_uint32), C.c_int64(len(rows)),
                                                C.c_uint32(num_bin), ptr(out, C.c_int64)))
    return out


def quantize(grad, hess, bins=4, stochastic=False, seed=0, const_hess=-1):
    """Returns (dequantized grad f32, dequantized hess f32, discretized i8[2n], scales)."""
    g = np.array(grad, dtype=np.float32, copy=True)
    h = np.array(hess, dtype=np.float32, copy=True)
    disc = np.zeros(2 * len(g), dtype=np.int8)
    scales = np.zeros(2, dtype=np.float64)
    _check(lib().oracle_quantize(ptr(g, C.c_float), ptr(h, C.c_float), C.c_int64(len(g)),
                                 C.c_int32(bins), C.c_int32(int(stochastic)),
                                 C.c_uint64(seed), C.c_int32(const_hess), ptr(disc, C.c_int8),
                                 ptr(scales, C.c_double)))
    return g, h, disc, scales


def xorshift_u01(state, n):
    out = np.zeros(n, dtype=np.float64)
    _check(lib().oracle_xorshift_u01(C.c_uint64(state), C.c_int64(n), ptr(out, C.c_double)))
    return out


def xorshift_states(state, n):
    """The raw xorshift64 states after 1..n steps of the discretizer's stream."""
    out = np.zeros(n, dtype=np.uint64)
    _check(lib().oracle_xorshift_states(C.c_uint64(state), C.c_int64(n), ptr(out, C.c_uint64)))
    return out


def fix_histogram(hist, num_bin, mfb, sum_g, sum_h):
    h = np.array(hist, dtype=np.float64, copy=True)
    _check(lib().oracle_fix_histogram(ptr(h, C.c_double), C.c_uint32(num_bin), C.c_uint32(mfb),
                                      C.c_double(sum_g), C.c_double(sum_h)))
    return h


def compact_histogram(hist, num_bin, offset):
    h = np.array(hist, dtype=np.float64, copy=True)
    _check(lib().oracle_compact_histogram(ptr(h, C.c_double), C.c_uint32(num_bin),
                                          C.c_int32(offset)))
    return h


def subtract(parent, child):
    p = np.ascontiguousarray(parent, dtype=np.float64)
    c = np.ascontiguousarray(child, dtype=np.float64)
    out = np.zeros_like(p)
    _check(lib().oracle_subtract(ptr(p, C.c_double), ptr(c, C.c_double), C.c_int64(len(p)),
                                 ptr(out, C.c_double)))
    return out


def find_best_split(hist, cfg, num_bin, offset, default_bin, skip_default_bin, na_as_missing,
                    run_forward, sum_gradient, sum_hessian, num_data):
    h = np.ascontiguousarray(hist, dtype=np.float64)
    out = SplitInfo()
    _check(lib().oracle_find_best_split(
        ptr(h, C.c_double), C.c_int64(len(h)), C.byref(cfg), C.c_uint32(num_bin),
        C.c_int32(offset), C.c_uint32(default_bin), C.c_int32(int(skip_default_bin)),
        C.c_int32(int(na_as_missing)), C.c_int32(int(run_forward)), C.c_double(sum_gradient),
        C.c_double(sum_hessian), C.c_int32(num_data), C.byref(out)))
    return out


def split_candidates(hist, cfg, num_bin, offset, default_bin, skip_default_bin, na_as_missing,
                     run_forward, sum_gradient, sum_hessian, num_data):
    """Every REVERSE / FORWARD candidate of one scan: its gain, or NaN where gated."""
    h = np.ascontiguousarray(hist, dtype=np.float64)
    cap = 2 * int(num_bin) + 2
    rev = np.zeros(cap, dtype=np.float64)
    fwd = np.zeros(cap, dtype=np.float64)
    nr, nf = C.c_int32(0), C.c_int32(0)
    _check(lib().oracle_split_candidates(
        ptr(h, C.c_double), C.c_int64(len(h)), C.byref(cfg), C.c_uint32(num_bin),
        C.c_int32(offset), C.c_uint32(default_bin), C.c_int32(int(skip_default_bin)),
        C.c_int32(int(na_as_missing)), C.c_int32(int(run_forward)), C.c_double(sum_gradient),
        C.c_double(sum_hessian), C.c_int32(num_data), ptr(rev, C.c_double), C.byref(nr),
        ptr(fwd, C.c_double), C.byref(nf), C.c_int32(cap)))
    return rev[:nr.value].copy(), fwd[:nf.value].copy()


def data_partition(bins, num_bin, min_bin, max_bin, threshold, mfb, na_as_missing=False,
                   default_left=False):
    b = np.ascontiguousarray(bins, dtype=np.uint32)
    order = np.zeros(len(b), dtype=np.uint32)
    lc = C.c_int64(0)
    _check(lib().oracle_data_partition(ptr(b, C.c_uint32), C.c_int64(len(b)), C.c_uint32(num_bin),
                                       C.c_uint32(min_bin), C.c_uint32(max_bin),
                                       C.c_uint32(threshold), C.c_uint32(mfb),
                                       C.c_int32(int(na_as_missing)),
                                       C.c_int32(int(default_left)), ptr(order, C.c_uint32),
                                       C.byref(lc)))
    return order, lc.value


def _bins_arg(bins_fm):
    b = np.ascontiguousarray(bins_fm)
    width = {np.dtype(np.uint8): 1, np.dtype(np.uint16): 2, np.dtype(np.uint32): 4}[b.dtype]
    return b, width


def _meta_arr(meta):
    arr = (FeatureMeta * len(meta))()
    for i, m in enumerate(meta):
        arr[i] = m
    return arr


def train_tree(bins_fm, meta, upper, grad, hess, cfg, num_leaves, max_depth=-1,
               feature_contri=None):
    """bins_fm: [F, N] u8/u16/u32 feature-major.  Returns (tree dict, layout).
    feature_contri: per-feature gain multipliers by real feature index (or None)."""
    b, width = _bins_arg(bins_fm)
    fc = None if feature_contri is None else np.ascontiguousarray(feature_contri, np.float64)
    F, N = b.shape
    marr = _meta_arr(meta)
    ub = None if upper is None else np.ascontiguousarray(upper, dtype=np.float64)
    g = np.ascontiguousarray(grad, dtype=np.float32)
    h = np.ascontiguousarray(hess, dtype=np.float32)
    tb = _tree_buffers(num_leaves, meta, upper)
    lb = LayoutBuffers(N, num_leaves)
    _check(lib().oracle_train_tree(b.ctypes.data_as(C.c_void_p), C.c_int32(width), C.c_int32(F),
                                   C.c_int64(N), marr, ptr(ub, C.c_double), ptr(g, C.c_float),
                                   ptr(h, C.c_float), C.byref(cfg), C.c_int32(num_leaves),
                                   C.c_int32(max_depth), ptr(fc, C.c_double),
                                   C.c_int32(0 if fc is None else len(fc)), C.byref(tb.out),
                                   C.byref(lb.out)))
    t = tb.to_dict()
    nl = t["num_leaves"]
    layout = {"indices": lb.indices, "leaf_begin": lb.leaf_begin[:nl].copy(),
              "leaf_count": lb.leaf_count[:nl].copy()}
    return t, layout


def binary_gradients(score, label):
    s = np.ascontiguousarray(score, dtype=np.float64)
    l = np.ascontiguousarray(label, dtype=np.float32)
    g = np.zeros(len(s), dtype=np.float32)
    h = np.zeros(len(s), dtype=np.float32)
    _check(lib().oracle_binary_gradients(ptr(s, C.c_double), ptr(l, C.c_float), ptr(g, C.c_float),
                                         ptr(h, C.c_float), C.c_int64(len(s))))
    return g, h


def boost_from_score(label):
    l = np.ascontiguousarray(label, dtype=np.float32)
    return lib().oracle_binary_boost_from_score(ptr(l, C.c_float), C.c_int64(len(l)))


def train_binary(bins_fm, meta, upper, label, cfg, num_leaves, max_depth, iters, lr,
                 boost_from_average=True, quantized=True, quant_bins=4, stochastic=True,
                 want_trees=True):
    b, width = _bins_arg(bins_fm)
    F, N = b.shape
    marr = _meta_arr(meta)
    ub = None if upper is None else np.ascontiguousarray(upper, dtype=np.float64)
    lab = np.ascontiguousarray(label, dtype=np.float32)
    scores = np.zeros(N, dtype=np.float64)
    trees = [_tree_buffers(num_leaves, meta, upper) for _ in range(iters)] if want_trees else []
    tarr = (type(trees[0].out) * iters)(*[t.out for t in trees]) if want_trees else None
    nt = C.c_int32(0)
    _check(lib().oracle_train_binary(
        b.ctypes.data_as(C.c_void_p), C.c_int32(width), C.c_int32(F), C.c_int64(N), marr,
        ptr(ub, C.c_double), ptr(lab, C.c_float), C.byref(cfg), C.c_int32(num_leaves),
        C.c_int32(max_depth), C.c_int32(iters), C.c_double(lr), C.c_int32(int(boost_from_average)),
        C.c_int32(int(quantized)), C.c_int32(quant_bins), C.c_int32(int(stochastic)),
        ptr(scores, C.c_double), tarr, C.byref(nt)))
    out_trees = []
    if want_trees:
        for i in range(nt.value):
            # copy back from the ctypes array element (struct copied by value)
            trees[i].out = tarr[i]
            out_trees.append(trees[i].to_dict())
    return scores, out_trees


def multiclass_gradients(score, label, num_class):
    """MulticlassSoftmax::get_gradients over class-major scores (K * n) -> (g, h)."""
    s = np.ascontiguousarray(score, dtype=np.float64)
    l = np.ascontiguousarray(label, dtype=np.float32)
    n = len(l)
    assert len(s) == n * num_class
    g = np.zeros(n * num_class, dtype=np.float32)
    h = np.zeros(n * num_class, dtype=np.float32)
    _check(lib().oracle_multiclass_gradients(ptr(s, C.c_double), ptr(l, C.c_float), C.c_int64(n),
                                             C.c_int32(num_class), ptr(g, C.c_float),
                                             ptr(h, C.c_float)))
    return g, h


def train_multiclass(bins_fm, meta, upper, label, num_class, cfg, num_leaves, max_depth, iters,
                     lr, boost_from_average=True, quantized=False, quant_bins=4, stochastic=True,
                     want_trees=True, quant_renew_leaf=False):
    """Softmax boosting: (class-major final scores [K * n], trees in iteration-major,
    class-minor order)."""
    b, width = _bins_arg(bins_fm)
    F, N = b.shape
    marr = _meta_arr(meta)
    ub = None if upper is None else np.ascontiguousarray(upper, dtype=np.float64)
    lab = np.ascontiguousarray(label, dtype=np.float32)
    scores = np.zeros(N * num_class, dtype=np.float64)
    cap = iters * num_class
    trees = [_tree_buffers(num_leaves, meta, upper) for _ in range(cap)] if want_trees else []
    tarr = (type(trees[0].out) * cap)(*[t.out for t in trees]) if want_trees else None
    nt = C.c_int32(0)
    _check(lib().oracle_train_multiclass(
        b.ctypes.data_as(C.c_void_p), C.c_int32(width), C.c_int32(F), C.c_int64(N), marr,
        ptr(ub, C.c_double), ptr(lab, C.c_float), C.c_int32(num_class), C.byref(cfg),
        C.c_int32(num_leaves), C.c_int32(max_depth), C.c_int32(iters), C.c_double(lr),
        C.c_int32(int(boost_from_average)), C.c_int32(int(quantized)), C.c_int32(quant_bins),
        C.c_int32(int(stochastic)), ptr(scores, C.c_double), tarr, C.byref(nt),
        C.c_int32(int(quant_renew_leaf))))
    out_trees = []
    if want_trees:
        for i in range(nt.value):
            trees[i].out = tarr[i]
            out_trees.append(trees[i].to_dict())
    return scores, out_trees


OBJECTIVE_BINARY, OBJECTIVE_REGRESSION, OBJECTIVE_LAMBDARANK = 0, 1, 2


class TrainParams(C.Structure):
    """oracle_train_params (lgbm_oracle.cpp)."""
    _fields_ = [("objective", C.c_int32), ("num_leaves", C.c_int32), ("max_depth", C.c_int32),
                ("iters", C.c_int32), ("learning_rate", C.c_double),
                ("boost_from_average", C.c_int32), ("quantized", C.c_int32),
                ("quant_bins", C.c_int32), ("stochastic", C.c_int32),
                ("feature_fraction", C.c_double), ("feature_fraction_seed", C.c_int32),
                ("lambdarank_norm", C.c_int32), ("sigmoid", C.c_double),
                ("truncation_level", C.c_int32), ("num_queries", C.c_int32),
                ("query_boundaries", C.POINTER(C.c_int32)),
                ("quant_renew_leaf", C.c_int32), ("_pad", C.c_int32)]


def train(bins_fm, meta, upper, label, cfg, objective, num_leaves, max_depth, iters, lr,
          boost_from_average=True, quantized=False, quant_bins=4, stochastic=True,
          feature_fraction=1.0, feature_fraction_seed=2, query_boundaries=None, sigmoid=1.0,
          lambdarank_norm=True, truncation_level=30, want_trees=True, quant_renew_leaf=False):
    """The one-tree-per-iteration boosting loop for binary logloss (0), L2 regression
    (1) or lambdarank (2, over `query_boundaries`), with the optional quantizer (and its
    quant_train_renew_leaf) and per-tree column sampling.  Returns (final scores,
    trees)."""
    b, width = _bins_arg(bins_fm)
    F, N = b.shape
    marr = _meta_arr(meta)
    ub = None if upper is None else np.ascontiguousarray(upper, dtype=np.float64)
    lab = np.ascontiguousarray(label, dtype=np.float32)
    qb = None if query_boundaries is None else np.ascontiguousarray(query_boundaries, np.int32)
    p = TrainParams()
    p.objective = objective
    p.num_leaves, p.max_depth, p.iters, p.learning_rate = num_leaves, max_depth, iters, lr
    p.boost_from_average, p.quantized = int(boost_from_average), int(quantized)
    p.quant_bins, p.stochastic = quant_bins, int(stochastic)
    p.feature_fraction, p.feature_fraction_seed = feature_fraction, feature_fraction_seed
    p.lambdarank_norm, p.sigmoid, p.truncation_level = int(lambdarank_norm), sigmoid, truncation_level
    p.num_queries = 0 if qb is None else len(qb) - 1
    p.query_boundaries = ptr(qb, C.c_int32) if qb is not None else None
    p.quant_renew_leaf = int(quant_renew_leaf)
    scores = np.zeros(N, dtype=np.float64)
    trees = [_tree_buffers(num_leaves, meta, upper) for _ in range(iters)] if want_trees else []
    tarr = (type(trees[0].out) * iters)(*[t.out for t in trees]) if want_trees else None
    nt = C.c_int32(0)
    _check(lib().oracle_train(b.ctypes.data_as(C.c_void_p), C.c_int32(width), C.c_int32(F),
                              C.c_int64(N), marr, ptr(ub, C.c_double), ptr(lab, C.c_float),
                              C.byref(cfg), C.byref(p), ptr(scores, C.c_double), tarr,
                              C.byref(nt)))
    out_trees = []
    if want_trees:
        for i in range(nt.value):
            trees[i].out = tarr[i]
            out_trees.append(trees[i].to_dict())
    return scores, out_trees


def regression_gradients(score, label):
    s = np.ascontiguousarray(score, dtype=np.float64)
    l = np.ascontiguousarray(label, dtype=np.float32)
    g = np.zeros(len(s), dtype=np.float32)
    h = np.zeros(len(s), dtype=np.float32)
    _check(lib().oracle_regression_gradients(ptr(s, C.c_double), ptr(l, C.c_float),
                                             C.c_int64(len(s)), ptr(g, C.c_float),
                                             ptr(h, C.c_float)))
    return g, h


def regression_boost_from_score(label):
    l = np.ascontiguousarray(label, dtype=np.float32)
    return lib().oracle_regression_boost_from_score(ptr(l, C.c_float), C.c_int64(len(l)))


def lambdarank_gradients(score, label, query_boundaries, sigmoid=1.0, norm=True,
                         truncation_level=30):
    s = np.ascontiguousarray(score, dtype=np.float64)
    l = np.ascontiguousarray(label, dtype=np.float32)
    qb = np.ascontiguousarray(query_boundaries, dtype=np.int32)
    g = np.zeros(len(s), dtype=np.float32)
    h = np.zeros(len(s), dtype=np.float32)
    _check(lib().oracle_lambdarank_gradients(
        ptr(s, C.c_double), ptr(l, C.c_float), C.c_int64(len(s)), ptr(qb, C.c_int32),
        C.c_int32(len(qb) - 1), C.c_double(sigmoid), C.c_int32(int(norm)),
        C.c_int32(truncation_level), ptr(g, C.c_float), ptr(h, C.c_float)))
    return g, h


def col_sampler_trace(feature_fraction, feature_fraction_bynode, seed, num_features, n_nodes):
    """(tree selection [nf] int8, node selections [n_nodes, nf] int8) of a fresh sampler."""
    bt = np.zeros(num_features, dtype=np.int8)
    nodes = np.zeros((max(n_nodes, 1), num_features), dtype=np.int8)
    _check(lib().oracle_col_sampler_trace(C.c_double(feature_fraction),
                                          C.c_double(feature_fraction_bynode), C.c_int32(seed),
                                          C.c_int32(num_features), C.c_int32(n_nodes),
                                          ptr(bt, C.c_int8), ptr(nodes, C.c_int8)))
    return bt, nodes[:n_nodes]


def random_sample(seed, n, k):
    out = np.zeros(max(k, 1), dtype=np.int32)
    ln = C.c_int32(0)
    _check(lib().oracle_random_sample(C.c_int32(seed), C.c_int32(n), C.c_int32(k),
                                      ptr(out, C.c_int32), C.byref(ln)))
    return out[:ln.value]
