"""ctypes mirrors of the structs declared in include/lgbm_hip.h.

Field order and widths must match the header exactly; tests/test_abi.py checks the
sizes and offsets against the compiled library's own view of them.
"""
import ctypes as C

import numpy as np

STATUS = {
    0: "OK",
    -1: "LENGTH_MISMATCH",
    -2: "BIN_INDEX_OUT_OF_RANGE",
    -3: "CAPABILITY_UNAVAILABLE",
    -4: "RUNTIME",
    -5: "HIP_ERROR",
    -6: "INVALID_ARGUMENT",
    -7: "INVALID_LEAF_HESSIAN",
}

MISSING_NONE, MISSING_ZERO, MISSING_NAN = 0, 1, 2


class GainConfig(C.Structure):
    """`GainConfig` (crates/lgbm-compute/src/gain.rs:904-960)."""

    _fields_ = [
        ("min_data_in_leaf", C.c_int32),
        ("_pad0", C.c_int32),
        ("min_sum_hessian_in_leaf", C.c_double),
        ("max_delta_step", C.c_double),
        ("lambda_l1", C.c_double),
        ("lambda_l2", C.c_double),
        ("min_gain_to_split", C.c_double),
        ("path_smooth", C.c_double),
        ("parent_output", C.c_double),
        ("min_data_per_group", C.c_int32),
        ("max_cat_threshold", C.c_int32),
        ("cat_l2", C.c_double),
        ("cat_smooth", C.c_double),
        ("max_cat_to_onehot", C.c_int32),
        ("_pad1", C.c_int32),
    ]

    @classmethod
    def make(cls, min_data_in_leaf=20, min_sum_hessian_in_leaf=1e-3, max_delta_step=0.0,
             lambda_l1=0.0, lambda_l2=0.0, min_gain_to_split=0.0, path_smooth=0.0):
        # Defaults are the config.h defaults (GainConfig::default, gain.rs:962-969).
        c = cls()
        c.min_data_in_leaf = min_data_in_leaf
        c.min_sum_hessian_in_leaf = min_sum_hessian_in_leaf
        c.max_delta_step = max_delta_step
        c.lambda_l1 = lambda_l1
        c.lambda_l2 = lambda_l2
        c.min_gain_to_split = min_gain_to_split
        c.path_smooth = path_smooth
        c.parent_output = 0.0
        c.min_data_per_group = 100
        c.max_cat_threshold = 32
        c.cat_l2 = 10.0
        c.cat_smooth = 10.0
        c.max_cat_to_onehot = 4
        return c


class SplitInfo(C.Structure):
    """`SplitInfo` (crates/lgbm-compute/src/gain.rs:1019-1053)."""

    _fields_ = [
        ("threshold", C.c_uint32),
        ("left_count", C.c_int32),
        ("right_count", C.c_int32),
        ("default_left", C.c_int32),
        ("gain", C.c_double),
        ("left_sum_gradient", C.c_double),
        ("left_sum_hessian", C.c_double),
        ("right_sum_gradient", C.c_double),
        ("right_sum_hessian", C.c_double),
        ("left_output", C.c_double),
        ("right_output", C.c_double),
    ]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class BatchedFeature(C.Structure):
    """`BatchedSplitFeature` (crates/lgbm-compute/src/kernels/split.rs:77-95)."""

    _fields_ = [
        ("slot_off", C.c_uint64),
        ("num_bin", C.c_uint32),
        ("offset", C.c_int32),
        ("default_bin", C.c_uint32),
        ("most_freq_bin", C.c_uint32),
        ("skip_default_bin", C.c_int32),
        ("na_as_missing", C.c_int32),
        ("run_forward", C.c_int32),
        ("_pad", C.c_int32),
    ]


class FeatureMeta(C.Structure):
    """Numeric `FeatureColumn` descriptors (crates/lgbm-treelearner/src/learner.rs:87-204)."""

    _fields_ = [
        ("num_bin", C.c_uint32),
        ("offset", C.c_int32),
        ("min_bin", C.c_uint32),
        ("max_bin", C.c_uint32),
        ("default_bin", C.c_uint32),
        ("most_freq_bin", C.c_uint32),
        ("missing_type", C.c_int32),
        ("real_feature_index", C.c_int32),
        ("bin_type", C.c_int32),
    ]


class TreeOut(C.Structure):
    _fields_ = [
        ("num_leaves", C.c_int32),
        ("_pad", C.c_int32),
        ("split_feature", C.POINTER(C.c_int32)),
        ("threshold_in_bin", C.POINTER(C.c_uint32)),
        ("threshold", C.POINTER(C.c_double)),
        ("split_gain", C.POINTER(C.c_float)),
        ("decision_type", C.POINTER(C.c_int8)),
        ("left_child", C.POINTER(C.c_int32)),
        ("right_child", C.POINTER(C.c_int32)),
        ("internal_value", C.POINTER(C.c_double)),
        ("internal_count", C.POINTER(C.c_int32)),
        ("leaf_value", C.POINTER(C.c_double)),
        ("leaf_weight", C.POINTER(C.c_double)),
        ("leaf_count", C.POINTER(C.c_int32)),
        ("leaf_depth", C.POINTER(C.c_int32)),
        ("leaf_parent", C.POINTER(C.c_int32)),
        ("internal_weight", C.POINTER(C.c_double)),
        ("num_cat", C.c_int32),
        ("cat_threshold_cap", C.c_int32),
        ("cat_boundaries", C.POINTER(C.c_int32)),
        ("cat_threshold", C.POINTER(C.c_uint32)),
    ]


class LeafSums(C.Structure):
    """lgbm_leaf_sums: a leaf's raw totals and its parent_output (LeafSplits)."""
    _fields_ = [("sum_gradient", C.c_double), ("sum_hessian", C.c_double),
                ("num_data", C.c_int32), ("_pad", C.c_int32), ("weight", C.c_double)]


class LayoutOut(C.Structure):
    _fields_ = [
        ("indices", C.POINTER(C.c_uint32)),
        ("leaf_begin", C.POINTER(C.c_int32)),
        ("leaf_count", C.POINTER(C.c_int32)),
    ]


def ptr(a, ctype):
    """Pointer to a contiguous numpy array (or None)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data_as(C.POINTER(ctype))


_TREE_FIELDS = [
    ("split_feature", np.int32, C.c_int32, "node"),
    ("threshold_in_bin", np.uint32, C.c_uint32, "node"),
    ("threshold", np.float64, C.c_double, "node"),
    ("split_gain", np.float32, C.c_float, "node"),
    ("decision_type", np.int8, C.c_int8, "node"),
    ("left_child", np.int32, C.c_int32, "node"),
    ("right_child", np.int32, C.c_int32, "node"),
    ("internal_value", np.float64, C.c_double, "node"),
    ("internal_count", np.int32, C.c_int32, "node"),
    ("leaf_value", np.float64, C.c_double, "leaf"),
    ("leaf_weight", np.float64, C.c_double, "leaf"),
    ("leaf_count", np.int32, C.c_int32, "leaf"),
    ("leaf_depth", np.int32, C.c_int32, "leaf"),
    ("leaf_parent", np.int32, C.c_int32, "leaf"),
    ("internal_weight", np.float64, C.c_double, "node"),
]


CAT_WORDS_PER_NODE = 64  # category bitset capacity per categorical node (2048 categories)


class TreeBuffers:
    """Host arrays backing one TreeOut (capacity num_leaves)."""

    def __init__(self, num_leaves, cat_words=None):
        """cat_words: capacity of cat_threshold in 32-bit words (default
        CAT_WORDS_PER_NODE per internal node)."""
        self.cap = num_leaves
        self.arrays = {}
        self.out = TreeOut()
        for name, dt, ct, kind in _TREE_FIELDS:
            n = max(num_leaves - 1, 1) if kind == "node" else num_leaves
            a = np.zeros(n, dtype=dt)
            self.arrays[name] = a
            setattr(self.out, name, ptr(a, ct))
        self.cat_boundaries = np.zeros(max(num_leaves, 2), dtype=np.int32)
        if cat_words is None:
            cat_words = max(num_leaves - 1, 1) * CAT_WORDS_PER_NODE
        self.cat_threshold = np.zeros(max(int(cat_words), 1), dtype=np.uint32)
        self.out.cat_boundaries = ptr(self.cat_boundaries, C.c_int32)
        self.out.cat_threshold = ptr(self.cat_threshold, C.c_uint32)
        self.out.cat_threshold_cap = len(self.cat_threshold)

    @classmethod
    def from_dict(cls, d):
        """A TreeOut over copies of a tree dict's arrays (as to_dict returns it)."""
        lens = [len(d[n]) + (1 if k == "node" else 0) for n, _, _, k in _TREE_FIELDS if n in d]
        tb = cls(max([int(d["num_leaves"]), 1] + lens))
        tb.out.num_leaves = int(d["num_leaves"])
        for name, dt, _, _ in _TREE_FIELDS:
            if name in d:
                v = np.asarray(d[name], dtype=dt)
                tb.arrays[name][:len(v)] = v
        nc = int(d.get("num_cat", 0))
        tb.out.num_cat = nc
        if nc:
            cb = np.asarray(d["cat_boundaries"], np.int32)
            ct = np.asarray(d["cat_threshold"], np.uint32)
            if len(ct) > len(tb.cat_threshold):
                tb.cat_threshold = np.zeros(len(ct), np.uint32)
                tb.out.cat_threshold = ptr(tb.cat_threshold, C.c_uint32)
                tb.out.cat_threshold_cap = len(ct)
            tb.cat_boundaries[:len(cb)] = cb
            tb.cat_threshold[:len(ct)] = ct
        return tb

    def to_dict(self):
        nl = self.out.num_leaves
        d = {"num_leaves": nl}
        for name, _, _, kind in _TREE_FIELDS:
            n = nl - 1 if kind == "node" else nl
            d[name] = self.arrays[name][:n].copy()
        nc = int(self.out.num_cat)
        d["num_cat"] = nc
        d["cat_boundaries"] = self.cat_boundaries[:nc + 1].copy() if nc else np.zeros(0, np.int32)
        d["cat_threshold"] = (self.cat_threshold[:self.cat_boundaries[nc]].copy() if nc
                              else np.zeros(0, np.uint32))
        return d


class LayoutBuffers:
    def __init__(self, num_data, num_leaves):
        self.indices = np.zeros(num_data, dtype=np.uint32)
        self.leaf_begin = np.zeros(num_leaves, dtype=np.int32)
        self.leaf_count = np.zeros(num_leaves, dtype=np.int32)
        self.out = LayoutOut(ptr(self.indices, C.c_uint32), ptr(self.leaf_begin, C.c_int32),
                             ptr(self.leaf_count, C.c_int32))
