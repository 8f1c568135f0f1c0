"""HipBackend — Python mirror of the reference's `Backend` seam over the C-ABI.

Method names follow `trait Backend` (crates/lgbm-compute/src/lib.rs:1092-2782) and
`GradientDiscretizer` (crates/lgbm-treelearner/src/gradient_discretizer.rs); every
call goes to lightgbm_rs_amd/liblgbm_hip.so.  There is no CPU fallback: if the
library or a HIP device is missing, construction raises.
"""
import ctypes as C
import os

import numpy as np

from ._abi import (STATUS, BatchedFeature, FeatureMeta, GainConfig, LayoutBuffers, LeafSums,
                   SplitInfo, TreeBuffers, ptr)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblgbm_hip.so")

_lib = None


class HipError(RuntimeError):
    """A non-zero status from the C-ABI (mirrors `ComputeError`, error.rs)."""

    def __init__(self, code, msg):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


def load_library():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
        _lib = C.CDLL(LIB_PATH)
    return _lib


def _feature_meta_array(meta):
    arr = (FeatureMeta * len(meta))()
    for i, m in enumerate(meta):
        arr[i] = m
    return arr


class HipBackend:
    """One device context (`GpuBackend` with its resident caches, lib.rs:3848-3934)."""

    def __init__(self, device=0):
        self.lib = load_library()
        self.ctx = C.c_void_p()
        rc = self.lib.lgbm_hip_ctx_create(C.c_int(device), C.byref(self.ctx))
        if rc != 0:
            raise HipError(rc, self._err(None))
        self.num_data = 0
        self.num_features = 0
        self.slot_len = 0

    def cat_threshold_words(self, num_leaves):
        """cat_threshold capacity a tree of num_leaves needs over the resident bins
        (lgbm_hip_cat_threshold_words)."""
        out = C.c_int64(0)
        self._check(self.lib.lgbm_hip_cat_threshold_words(self.ctx, C.c_int32(num_leaves),
                                                          C.byref(out)))
        return int(out.value)

    def _tree_buffers(self, num_leaves, fresh=False):
        """Host arrays for one grown tree, reused across calls (to_dict copies);
        fresh=True: new arrays (several trees filled by one call).  The categorical
        bitset capacity covers the resident bins' widest category set per node."""
        words = max(self.cat_threshold_words(num_leaves), max(num_leaves - 1, 1) * 64)
        if fresh:
            return TreeBuffers(num_leaves, words)
        cache = self.__dict__.setdefault("_tb_cache", {})
        key = (num_leaves, words)
        if key not in cache:
            cache[key] = TreeBuffers(num_leaves, words)
        return cache[key]

    def _err(self, ctx):
        buf = C.create_string_buffer(1024)
        self.lib.lgbm_hip_last_error(ctx, buf, C.c_size_t(1024))
        return buf.value.decode()

    def _check(self, rc):
        if rc != 0:
            raise HipError(rc, self._err(self.ctx))

    def close(self):
        if self.ctx:
            self.lib.lgbm_hip_ctx_destroy(self.ctx)
            self.ctx = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- resident data -------------------------------------------------------
    def upload_resident_bins(self, bins_feature_major, meta, bin_upper_bound=None):
        """`Backend::upload_resident_bins` (lib.rs:1564): bins [F, N] u8, or u16
        (lgbm_hip_upload_bins16) when given as uint16."""
        marr = _feature_meta_array(meta)
        ub = None if bin_upper_bound is None else np.ascontiguousarray(bin_upper_bound, np.float64)
        if np.asarray(bins_feature_major).dtype == np.uint16:
            b = np.ascontiguousarray(bins_feature_major, dtype=np.uint16)
            F, N = b.shape
            self._check(self.lib.lgbm_hip_upload_bins16(self.ctx, ptr(b, C.c_uint16), C.c_int32(F),
                                                        C.c_int64(N), marr, ptr(ub, C.c_double)))
        else:
            b = np.ascontiguousarray(bins_feature_major, dtype=np.uint8)
            F, N = b.shape
            self._check(self.lib.lgbm_hip_upload_bins(self.ctx, ptr(b, C.c_uint8), C.c_int32(F),
                                                      C.c_int64(N), marr, ptr(ub, C.c_double)))
        self.num_data, self.num_features = N, F
        self.slot_len = 2 * sum(m.num_bin for m in meta)

    def upload_resident_grad_hess(self, grad, hess):
        """`Backend::upload_resident_grad_hess` (lib.rs:1607)."""
        g = np.ascontiguousarray(grad, dtype=np.float32)
        h = np.ascontiguousarray(hess, dtype=np.float32)
        self._check(self.lib.lgbm_hip_set_gradients(self.ctx, ptr(g, C.c_float), ptr(h, C.c_float),
                                                    C.c_int64(len(g))))

    def discretize_dequantize_in_place(self, num_grad_quant_bins=4, stochastic=True, seed=0,
                                       want_values=False):
        """`GradientDiscretizer::discretize_dequantize_in_place` on the resident g/h.

        Returns (scales, dequantized grad, dequantized hess) — the last two only
        when want_values."""
        n = self.num_data
        dg = np.zeros(n, np.float32) if want_values else None
        dh = np.zeros(n, np.float32) if want_values else None
        scales = np.zeros(2, np.float64)
        self._check(self.lib.lgbm_hip_quantize(self.ctx, C.c_int32(num_grad_quant_bins),
                                               C.c_int32(int(stochastic)), C.c_uint64(seed),
                                               ptr(dg, C.c_float), ptr(dh, C.c_float),
                                               ptr(scales, C.c_double)))
        return scales, dg, dh

    def set_dequantized_grad_hess(self, grad, hess, num_grad_quant_bins=4, grad_scale=0.0,
                                  hess_scale=0.0):
        """The quantized pairs recovered exactly from dequantized values f32(q * scale)
        (the arrays quantize_grad_hess_in_place leaves, gbdt.rs:43-62); scales <= 0
        take the last discretize_dequantize_in_place's."""
        g = np.ascontiguousarray(grad, dtype=np.float32)
        h = np.ascontiguousarray(hess, dtype=np.float32)
        self._check(self.lib.lgbm_hip_set_dequantized_gradients(
            self.ctx, ptr(g, C.c_float), ptr(h, C.c_float), C.c_int64(len(g)),
            C.c_int32(num_grad_quant_bins), C.c_double(grad_scale), C.c_double(hess_scale)))

    def set_feature_contri(self, contri=None):
        """config.feature_contri gain multipliers by real feature index (None: reset)."""
        c = None if contri is None else np.ascontiguousarray(contri, dtype=np.float64)
        self._check(self.lib.lgbm_hip_set_feature_contri(self.ctx, ptr(c, C.c_double),
                                                         C.c_int32(0 if c is None else len(c))))

    def discretized(self):
        """The `discretize` buffer: out[2i] = hess, out[2i+1] = grad (i8)."""
        out = np.zeros(2 * self.num_data, np.int8)
        self._check(self.lib.lgbm_hip_get_discretized(self.ctx, ptr(out, C.c_int8),
                                                      C.c_int64(self.num_data)))
        return out

    # ---- per-op seam ---------------------------------------------------------
    def construct_int_histogram(self, leaf_rows=None):
        """Exact integer histogram of the quantized gradients (all features)."""
        rows = None if leaf_rows is None else np.ascontiguousarray(leaf_rows, np.uint32)
        out = np.zeros(self.slot_len, np.int64)
        self._check(self.lib.lgbm_hip_build_int_histogram(
            self.ctx, ptr(rows, C.c_uint32), C.c_int64(0 if rows is None else len(rows)),
            ptr(out, C.c_int64)))
        return out

    # ---- device-resident histogram slots (lib.rs:1940-2058) -------------------------
    def reset_resident_pool(self, num_slots, slot_len=None):
        """`Backend::reset_resident_pool`: num_slots device slots of slot_len doubles."""
        self._check(self.lib.lgbm_hip_resident_reset(
            self.ctx, C.c_int32(num_slots), C.c_int64(self.slot_len if slot_len is None else slot_len)))

    def move_resident(self, src_slot, dst_slot):
        """`Backend::move_resident`."""
        self._check(self.lib.lgbm_hip_resident_move(self.ctx, C.c_int32(src_slot), C.c_int32(dst_slot)))

    def subtract_resident(self, parent_slot, smaller_slot, larger_slot):
        """`Backend::subtract_resident`: larger = parent - smaller on the device."""
        self._check(self.lib.lgbm_hip_resident_subtract(self.ctx, C.c_int32(parent_slot),
                                                        C.c_int32(smaller_slot),
                                                        C.c_int32(larger_slot)))

    def scan_resident_leaf(self, slot, feats, cfg, sum_gradient, sum_hessian, num_data):
        """`Backend::scan_resident_leaf`: per-feature SplitInfos of a resident slot."""
        farr = (BatchedFeature * len(feats))(*feats)
        out = (SplitInfo * len(feats))()
        self._check(self.lib.lgbm_hip_resident_scan(
            self.ctx, C.c_int32(slot), farr, C.c_int32(len(feats)), C.byref(cfg),
            C.c_double(sum_gradient), C.c_double(sum_hessian), C.c_int32(num_data), out))
        return list(out)

    def scan_resident_siblings(self, smaller_slot, larger_slot, feats, cfg, smaller_totals,
                               larger_totals):
        """`Backend::scan_resident_siblings`; totals = (sum_g, sum_h, num_data,
        parent_output) of each sibling.  Returns (smaller splits, larger splits)."""
        farr = (BatchedFeature * len(feats))(*feats)
        o1 = (SplitInfo * len(feats))()
        o2 = (SplitInfo * len(feats))()
        st, lt = LeafSums(), LeafSums()
        st.sum_gradient, st.sum_hessian, st.num_data, st.weight = smaller_totals
        lt.sum_gradient, lt.sum_hessian, lt.num_data, lt.weight = larger_totals
        self._check(self.lib.lgbm_hip_resident_scan_siblings(
            self.ctx, C.c_int32(smaller_slot), C.c_int32(larger_slot), farr, C.c_int32(len(feats)),
            C.byref(cfg), C.byref(st), C.byref(lt), o1, o2))
        return list(o1), list(o2)

    def read_resident(self, slot):
        """A slot's histogram as host doubles (lgbm_hip_resident_read)."""
        out = np.zeros(self.slot_len, np.float64)
        self._check(self.lib.lgbm_hip_resident_read(self.ctx, C.c_int32(slot), ptr(out, C.c_double)))
        return out

    def build_resident_leaf(self, leaf_rows, sum_gradient, sum_hessian, slot=None):
        """`Backend::build_resident_leaf` (lib.rs:1953-1972): build + fix + compact.
        slot given: into that resident slot (nothing returned); else the histogram is
        returned as host doubles."""
        rows = None if leaf_rows is None else np.ascontiguousarray(leaf_rows, np.uint32)
        if slot is not None:
            self._check(self.lib.lgbm_hip_resident_build(
                self.ctx, C.c_int32(slot), ptr(rows, C.c_uint32),
                C.c_int64(0 if rows is None else len(rows)), C.c_double(sum_gradient),
                C.c_double(sum_hessian)))
            return None
        out = np.zeros(self.slot_len, np.float64)
        self._check(self.lib.lgbm_hip_build_leaf_histogram(
            self.ctx, ptr(rows, C.c_uint32), C.c_int64(0 if rows is None else len(rows)),
            C.c_double(sum_gradient), C.c_double(sum_hessian), ptr(out, C.c_double)))
        return out

    def find_best_splits_batched(self, hist, feats, cfg, sum_gradient, sum_hessian, num_data):
        """`Backend::find_best_splits_batched` (lib.rs:1500-1548)."""
        h = np.ascontiguousarray(hist, np.float64)
        farr = (BatchedFeature * len(feats))(*feats)
        out = (SplitInfo * len(feats))()
        self._check(self.lib.lgbm_hip_find_best_splits(
            self.ctx, ptr(h, C.c_double), C.c_int64(len(h)), farr, C.c_int32(len(feats)),
            C.byref(cfg), C.c_double(sum_gradient), C.c_double(sum_hessian), C.c_int32(num_data),
            out))
        return list(out)

    def subtract_histograms(self, parent, child):
        """`Backend::subtract_histograms` (lib.rs:1314)."""
        p = np.ascontiguousarray(parent, np.float64)
        c = np.ascontiguousarray(child, np.float64)
        out = np.zeros_like(p)
        self._check(self.lib.lgbm_hip_subtract_histograms(self.ctx, ptr(p, C.c_double),
                                                          ptr(c, C.c_double), C.c_int64(len(p)),
                                                          ptr(out, C.c_double)))
        return out

    def data_partition(self, bins, num_bin, min_bin, max_bin, threshold, most_freq_bin,
                       na_as_missing=False, default_left=False):
        """`Backend::data_partition` (lib.rs:1206) -> (order, split_point)."""
        b = np.ascontiguousarray(bins, np.uint32)
        order = np.zeros(len(b), np.uint32)
        lc = C.c_int64(0)
        self._check(self.lib.lgbm_hip_data_partition(
            self.ctx, ptr(b, C.c_uint32), C.c_int64(len(b)), C.c_uint32(num_bin),
            C.c_uint32(min_bin), C.c_uint32(max_bin), C.c_uint32(threshold),
            C.c_uint32(most_freq_bin), C.c_int32(int(na_as_missing)),
            C.c_int32(int(default_left)), ptr(order, C.c_uint32), C.byref(lc)))
        return order, lc.value

    # ---- coarse seam -----------------------------------------------------------
    def grow_tree_on_device_with_cfg(self, cfg, num_leaves, max_depth=-1, want_layout=True):
        """`Backend::grow_tree_on_device_with_cfg` (lib.rs:2771) -> (tree, layout)."""
        tb = self._tree_buffers(num_leaves)
        lb = LayoutBuffers(self.num_data, num_leaves) if want_layout else None
        self._check(self.lib.lgbm_hip_grow_tree(self.ctx, C.byref(cfg), C.c_int32(num_leaves),
                                                C.c_int32(max_depth), C.byref(tb.out),
                                                C.byref(lb.out) if lb else None))
        t = tb.to_dict()
        layout = None
        if lb is not None:
            nl = t["num_leaves"]
            layout = {"indices": lb.indices, "leaf_begin": lb.leaf_begin[:nl].copy(),
                      "leaf_count": lb.leaf_count[:nl].copy()}
        return t, layout

    # ---- boosting on device ------------------------------------------------------
    def set_labels(self, labels, init_score=0.0):
        lab = np.ascontiguousarray(labels, np.float32)
        self._check(self.lib.lgbm_hip_set_labels(self.ctx, ptr(lab, C.c_float), C.c_int64(len(lab)),
                                                 C.c_double(init_score)))
        self.num_class = 1

    def train_iter_binary(self, it, cfg, num_leaves, max_depth, learning_rate,
                          num_grad_quant_bins=4, stochastic=True, want_tree=True):
        tb = self._tree_buffers(num_leaves) if want_tree else None
        self._check(self.lib.lgbm_hip_train_iter_binary(
            self.ctx, C.c_int32(it), C.byref(cfg), C.c_int32(num_leaves), C.c_int32(max_depth),
            C.c_double(learning_rate), C.c_int32(num_grad_quant_bins), C.c_int32(int(stochastic)),
            C.byref(tb.out) if tb else None))
        return tb.to_dict() if tb else None

    # objectives other than binary (lgbm_hip_set_objective / lgbm_hip_train_iter)
    OBJECTIVES = {"binary": 0, "regression": 1, "lambdarank": 2}

    def set_objective(self, objective):
        self._check(self.lib.lgbm_hip_set_objective(self.ctx, C.c_int32(self.OBJECTIVES[objective])))

    def set_lambdarank(self, query_boundaries, sigmoid=1.0, norm=True, truncation_level=30):
        """LambdaRank over the resident labels (lgbm_hip_set_lambdarank)."""
        qb = np.ascontiguousarray(query_boundaries, np.int32)
        self._check(self.lib.lgbm_hip_set_lambdarank(
            self.ctx, ptr(qb, C.c_int32), C.c_int32(len(qb) - 1), C.c_double(sigmoid),
            C.c_int32(int(norm)), C.c_int32(truncation_level)))

    def set_col_sampler(self, feature_fraction, feature_fraction_bynode=1.0, seed=2):
        """Per-tree column sampling (lgbm_hip_set_col_sampler)."""
        self._check(self.lib.lgbm_hip_set_col_sampler(self.ctx, C.c_double(feature_fraction),
                                                      C.c_double(feature_fraction_bynode),
                                                      C.c_int32(seed)))

    def train_iter(self, it, cfg, num_leaves, max_depth, learning_rate, num_grad_quant_bins=4,
                   stochastic=True, want_tree=True):
        """One iteration of the context's objective (lgbm_hip_train_iter)."""
        tb = self._tree_buffers(num_leaves) if want_tree else None
        self._check(self.lib.lgbm_hip_train_iter(
            self.ctx, C.c_int32(it), C.byref(cfg), C.c_int32(num_leaves), C.c_int32(max_depth),
            C.c_double(learning_rate), C.c_int32(num_grad_quant_bins), C.c_int32(int(stochastic)),
            C.byref(tb.out) if tb else None))
        return tb.to_dict() if tb else None

    def set_labels_multiclass(self, labels, num_class, init_scores=None):
        """Class labels + the class-major score reset to init_scores[k] per class
        (lgbm_hip_set_labels_multiclass)."""
        lab = np.ascontiguousarray(labels, np.float32)
        init = None if init_scores is None else np.ascontiguousarray(init_scores, np.float64)
        self._check(self.lib.lgbm_hip_set_labels_multiclass(
            self.ctx, ptr(lab, C.c_float), C.c_int64(len(lab)), C.c_int32(num_class),
            ptr(init, C.c_double)))
        self.num_class = int(num_class)

    def train_iter_multiclass(self, it, cfg, num_leaves, max_depth, learning_rate,
                              num_grad_quant_bins=0, stochastic=True, class_need_train=None,
                              want_trees=True):
        """One softmax iteration (lgbm_hip_train_iter_multiclass): the num_class shrunk
        trees (num_leaves 0 for a class skipped by class_need_train)."""
        K = self.num_class
        tbs = [self._tree_buffers(num_leaves, fresh=True) for _ in range(K)] if want_trees else None
        arr = None
        if tbs:
            arr = (type(tbs[0].out) * K)(*[t.out for t in tbs])
        need = None if class_need_train is None else np.ascontiguousarray(class_need_train, np.int32)
        self._check(self.lib.lgbm_hip_train_iter_multiclass(
            self.ctx, C.c_int32(it), C.byref(cfg), C.c_int32(num_leaves), C.c_int32(max_depth),
            C.c_double(learning_rate), C.c_int32(num_grad_quant_bins), C.c_int32(int(stochastic)),
            ptr(need, C.c_int32), arr))
        if not tbs:
            return None
        out = []
        for k, tb in enumerate(tbs):
            tb.out = arr[k]
            out.append(tb.to_dict())
        return out

    def multiclass_gradients(self):
        """The device's class-major f32 (grad, hess) of the last softmax evaluation."""
        n = self.num_class * self.num_data
        g = np.zeros(n, np.float32)
        h = np.zeros(n, np.float32)
        self._check(self.lib.lgbm_hip_get_multiclass_gradients(
            self.ctx, ptr(g, C.c_float), ptr(h, C.c_float), C.c_int64(n)))
        return g, h

    def gradients(self):
        """The device's f32 (grad, hess) of the last objective evaluation."""
        g = np.zeros(self.num_data, np.float32)
        h = np.zeros(self.num_data, np.float32)
        self._check(self.lib.lgbm_hip_get_gradients(self.ctx, ptr(g, C.c_float), ptr(h, C.c_float),
                                                    C.c_int64(self.num_data)))
        return g, h

    def set_quant_renew_leaf(self, enable=True):
        """quant_train_renew_leaf: quantized trees' leaf outputs from the original
        gradients (lgbm_hip_set_quant_renew_leaf)."""
        self._check(self.lib.lgbm_hip_set_quant_renew_leaf(self.ctx, C.c_int32(int(enable))))

    def set_lookahead(self, enable=True):
        """Enqueue the next iteration's gradients + quantization inside
        train_iter_binary (lgbm_hip_set_lookahead); results are unchanged."""
        self._check(self.lib.lgbm_hip_set_lookahead(self.ctx, C.c_int32(int(enable))))

    def scores(self):
        """The resident training score (class-major [num_class * num_data] for multiclass)."""
        out = np.zeros(getattr(self, "num_class", 1) * self.num_data, np.float64)
        self._check(self.lib.lgbm_hip_get_scores(self.ctx, ptr(out, C.c_double),
                                                 C.c_int64(len(out))))
        return out

    def set_timing(self, enable=True):
        self._check(self.lib.lgbm_hip_set_timing(self.ctx, C.c_int32(int(enable))))

    def timing(self):
        """Per-family device ms (HIP events) and row counters since set_timing."""
        st = np.zeros(23, np.float64)
        self._check(self.lib.lgbm_hip_get_stats(self.ctx, ptr(st, C.c_double)))
        keys = ["hist_ms", "partition_ms", "scan_ms", "quant_ms", "objective_ms", "root_rows",
                "hist_launches", "partition_rows", "partition_launches", "record_bytes",
                "features", "cells", "partition_jobs", "rounds", "trees", "extra_rounds",
                "bin_ms", "bin_launches", "bin_values", "predict_ms", "predict_launches",
                "predict_walks", "hist_child_rows"]
        return {k: float(v) for k, v in zip(keys, st)}


def binary_boost_from_score(labels, sigmoid=1.0):
    """BinaryLogloss::boost_from_score (lgbm-objective/src/binary.rs:178-192)."""
    lib = load_library()
    lab = np.ascontiguousarray(labels, np.float32)
    out = C.c_double(0.0)
    rc = lib.lgbm_hip_binary_boost_from_score(ptr(lab, C.c_float), C.c_int64(len(lab)),
                                              C.c_double(sigmoid), C.byref(out))
    if rc != 0:
        raise HipError(rc, "boost_from_score: bad arguments")
    return out.value


def boost_from_score(objective, labels):
    """The objective's BoostFromScore (lgbm_hip_boost_from_score): binary log-odds,
    the L2 label mean, 0 for lambdarank."""
    lib = load_library()
    lab = np.ascontiguousarray(labels, np.float32)
    out = C.c_double(0.0)
    rc = lib.lgbm_hip_boost_from_score(C.c_int32(HipBackend.OBJECTIVES[objective]),
                                       ptr(lab, C.c_float), C.c_int64(len(lab)), C.byref(out))
    if rc != 0:
        raise HipError(rc, "boost_from_score: bad arguments")
    return out.value


PREDICT_KINDS = {"raw": 0, "transformed": 1, "leaf": 2, "contrib": 3}


class Model:
    """A LightGBM v4 model text parsed by the library (`model_text::load`,
    crates/lgbm-model/src/model_text.rs:48-160); host only, no device needed."""

    def __init__(self, text):
        self.lib = load_library()
        data = text.encode() if isinstance(text, str) else bytes(text)
        self.handle = C.c_void_p()
        self._check(self.lib.lgbm_hip_model_load(C.c_char_p(data), C.c_int64(len(data)),
                                                 C.byref(self.handle)))
        self._info()

    def _check(self, rc):
        if rc != 0:
            buf = C.create_string_buffer(1024)
            self.lib.lgbm_hip_model_last_error(buf, C.c_size_t(1024))
            raise HipError(rc, buf.value.decode())

    @classmethod
    def create(cls, num_class=1, num_tree_per_iteration=None, max_feature_idx=0,
               objective=None, feature_names=None, feature_infos=None):
        """An empty model to append grown trees to (the boosting loop's GbdtModel,
        crates/lgbm-boosting/src/gbdt.rs:1094-1140)."""
        self = cls.__new__(cls)
        self.lib = load_library()
        self.handle = C.c_void_p()
        enc = lambda v: None if v is None else C.c_char_p(v.encode())
        ntpi = num_class if num_tree_per_iteration is None else num_tree_per_iteration
        self._check(self.lib.lgbm_hip_model_create(
            C.c_int32(num_class), C.c_int32(ntpi), C.c_int32(max_feature_idx), enc(objective),
            enc(feature_names), enc(feature_infos), C.byref(self.handle)))
        self._info()
        return self

    def add_tree(self, tree, shrinkage=1.0, bias=0.0):
        """Append a grown tree dict (HipBackend.train_iter_binary / grow_tree_*):
        values already shrunk, `shrinkage` recorded, `bias` added to every value
        (Tree::add_bias, crates/lgbm-model/src/tree.rs:1161)."""
        tb = TreeBuffers.from_dict(tree)
        self._check(self.lib.lgbm_hip_model_add_tree(self.handle, C.byref(tb.out),
                                                     C.c_double(shrinkage), C.c_double(bias)))
        self._info()

    def to_text(self):
        """The model text (model_text::save, crates/lgbm-model/src/model_text.rs:216-320)."""
        need = C.c_size_t(0)
        self._check(self.lib.lgbm_hip_model_to_text(self.handle, None, C.c_size_t(0),
                                                    C.byref(need)))
        buf = C.create_string_buffer(need.value)
        self._check(self.lib.lgbm_hip_model_to_text(self.handle, buf, need, C.byref(need)))
        return buf.raw[:need.value - 1].decode()

    def _info(self):
        info = np.zeros(6, np.int64)
        self.lib.lgbm_hip_model_info(self.handle, ptr(info, C.c_int64))
        (self.num_trees, self.num_class, self.num_tree_per_iteration, self.max_feature_idx,
         self.num_iterations, self.objective) = (int(x) for x in info)

    @classmethod
    def from_file(cls, path):
        with open(path, "rb") as f:
            return cls(f.read())

    def close(self):
        if self.handle:
            self.lib.lgbm_hip_model_free(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _predict_shape(model, kind, rows, start_iteration, num_iteration):
    total = model.num_iterations
    start = min(max(start_iteration, 0), total)
    num = min(num_iteration, total - start) if num_iteration > 0 else total - start
    if kind == "leaf":
        width = num * model.num_tree_per_iteration
    elif kind == "contrib":
        width = model.num_tree_per_iteration * (model.max_feature_idx + 2)
    else:
        width = model.num_tree_per_iteration
    return (rows, width)


def _predict(self, model, X, kind="raw", start_iteration=0, num_iteration=-1):
    """predict_raw_mat_range / predict_mat / predict_leaf_index_mat / predict_contrib_mat
    (crates/lgbm-model/src/predict.rs:75-131, 378-485, 675-697) on the device: X is a
    dense [rows, cols] float32 matrix; returns float64 [rows, outputs], int32
    [rows, trees] ("leaf") or float64 [rows, classes * (max_feature_idx + 2)]
    ("contrib": per class the feature contributions then the expected value)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    rows, cols = X.shape
    shape = _predict_shape(model, kind, rows, start_iteration, num_iteration)
    out = np.zeros(shape, np.int32 if kind == "leaf" else np.float64)
    self._check(self.lib.lgbm_hip_predict(
        self.ctx, model.handle, ptr(X, C.c_float), C.c_int64(rows), C.c_int32(cols),
        C.c_int32(start_iteration), C.c_int32(num_iteration), C.c_int32(PREDICT_KINDS[kind]),
        out.ctypes.data_as(C.c_void_p)))
    return out


def _predict_device(self, model, x_ptr, rows, cols, out_ptr, kind="raw", start_iteration=0,
                    num_iteration=-1):
    """The same over device-resident buffers (raw device pointers, e.g. torch tensors'
    data_ptr())."""
    self._check(self.lib.lgbm_hip_predict_device(
        self.ctx, model.handle, C.c_void_p(x_ptr), C.c_int64(rows), C.c_int32(cols),
        C.c_int32(start_iteration), C.c_int32(num_iteration), C.c_int32(PREDICT_KINDS[kind]),
        C.c_void_p(out_ptr)))


def _predict_early_stop(self, model, X, freq, margin, start_iteration=0, num_iteration=-1):
    """predict_raw_early_stop_mat (crates/lgbm-model/src/predict.rs:557-605) on the
    device: (raw float64 [rows, num_tree_per_iteration], iterations int32 [rows])."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    rows, cols = X.shape
    out = np.zeros((rows, model.num_tree_per_iteration), np.float64)
    iters = np.zeros(rows, np.int32)
    self._check(self.lib.lgbm_hip_predict_early_stop(
        self.ctx, model.handle, ptr(X, C.c_float), C.c_int64(rows), C.c_int32(cols),
        C.c_int32(start_iteration), C.c_int32(num_iteration), C.c_int32(freq),
        C.c_double(margin), ptr(out, C.c_double), ptr(iters, C.c_int32)))
    return out, iters


def _predict_csr(self, model, indptr, indices, values, num_cols, kind="raw", start_iteration=0,
                 num_iteration=-1):
    """predict_raw_csr_range / predict_csr / predict_leaf_index_csr / predict_contrib_csr
    (crates/lgbm-model/src/predict.rs:132-160, 405-500, 699-722) on the device: a CSR
    matrix (indptr int64 [rows + 1], indices int32, values float32) of num_cols columns;
    returns what `predict` returns for the same rows made dense."""
    indptr = np.ascontiguousarray(indptr, dtype=np.int64)
    indices = np.ascontiguousarray(indices, dtype=np.int32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    if indices.shape != values.shape:
        raise ValueError("indices and values differ in length")
    rows = len(indptr) - 1
    shape = _predict_shape(model, kind, rows, start_iteration, num_iteration)
    out = np.zeros(shape, np.int32 if kind == "leaf" else np.float64)
    self._check(self.lib.lgbm_hip_predict_csr(
        self.ctx, model.handle, ptr(indptr, C.c_int64), ptr(indices, C.c_int32),
        ptr(values, C.c_float), C.c_int64(len(values)), C.c_int64(rows), C.c_int32(num_cols),
        C.c_int32(start_iteration), C.c_int32(num_iteration), C.c_int32(PREDICT_KINDS[kind]),
        out.ctypes.data_as(C.c_void_p)))
    return out


def _predict_csc(self, model, indptr, indices, values, num_rows, kind="raw", start_iteration=0,
                 num_iteration=-1):
    """predict_raw_csc_range / predict_csc / predict_leaf_index_csc / predict_contrib_csc
    (crates/lgbm-model/src/predict.rs:209-240) on the device: a CSC matrix (indptr int64
    [cols + 1], row indices int32, values float32) of num_rows rows."""
    indptr = np.ascontiguousarray(indptr, dtype=np.int64)
    indices = np.ascontiguousarray(indices, dtype=np.int32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    if indices.shape != values.shape:
        raise ValueError("indices and values differ in length")
    shape = _predict_shape(model, kind, num_rows, start_iteration, num_iteration)
    out = np.zeros(shape, np.int32 if kind == "leaf" else np.float64)
    self._check(self.lib.lgbm_hip_predict_csc(
        self.ctx, model.handle, ptr(indptr, C.c_int64), ptr(indices, C.c_int32),
        ptr(values, C.c_float), C.c_int64(len(values)), C.c_int64(num_rows),
        C.c_int32(len(indptr) - 1), C.c_int32(start_iteration), C.c_int32(num_iteration),
        C.c_int32(PREDICT_KINDS[kind]), out.ctypes.data_as(C.c_void_p)))
    return out


HipBackend.predict = _predict
HipBackend.predict_csc = _predict_csc
HipBackend.predict_csr = _predict_csr
HipBackend.predict_early_stop = _predict_early_stop
HipBackend.predict_device = _predict_device


def feature_meta(num_bin, most_freq_bin=0, missing_type=0, default_bin=None, real_index=0,
                 min_bin=0, max_bin=None, bin_type=0):
    """FeatureColumn descriptors with the offset rule of offset_for_most_freq_bin
    (lgbm-treelearner/src/lib.rs:89-95); bin_type 1: categorical."""
    m = FeatureMeta()
    m.num_bin = num_bin
    m.offset = 1 if most_freq_bin == 0 else 0
    m.min_bin = min_bin
    m.max_bin = num_bin - 1 if max_bin is None else max_bin
    m.default_bin = num_bin if default_bin is None else default_bin
    m.most_freq_bin = most_freq_bin
    m.missing_type = missing_type
    m.real_feature_index = real_index
    m.bin_type = bin_type
    return m


__all__ = ["HipBackend", "HipError", "GainConfig", "Model", "binary_boost_from_score",
           "feature_meta", "load_library"]
