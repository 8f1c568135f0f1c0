"""Feature binning: BinMapper construction on the host, value -> bin on the device.

Mirrors the reference's `BinMapper` (crates/lgbm-dataset/src/bin_mapper.rs) and the
booster's feature-column construction (crates/lgbm/src/booster.rs:449-520); every
call goes to lightgbm_rs_amd/liblgbm_hip.so.
"""
import ctypes as C

import numpy as np

from .backend import HipBackend, HipError, load_library

DEFAULTS = dict(max_bin=255, min_data_in_bin=3, min_data_in_leaf=20, pre_filter=False,
                use_missing=True, zero_as_missing=False, bin_construct_sample_cnt=200000,
                data_random_seed=1)
MISSING = {0: "none", 1: "zero", 2: "nan"}


class BinParams(C.Structure):
    _fields_ = [(k, C.c_int32) for k in ("max_bin", "min_data_in_bin", "min_data_in_leaf",
                                         "pre_filter", "use_missing", "zero_as_missing",
                                         "bin_construct_sample_cnt", "data_random_seed")]

    @classmethod
    def make(cls, **kw):
        unknown = set(kw) - set(DEFAULTS)
        if unknown:
            raise TypeError(f"unknown binning parameters: {sorted(unknown)}")
        v = dict(DEFAULTS, **kw)
        return cls(*(int(v[k]) for k, _ in cls._fields_))


class BinMapperInfo(C.Structure):
    _fields_ = [("num_bin", C.c_int32), ("missing_type", C.c_int32), ("bin_type", C.c_int32),
                ("is_trivial", C.c_int32), ("default_bin", C.c_uint32),
                ("most_freq_bin", C.c_uint32), ("sparse_rate", C.c_double),
                ("min_val", C.c_double), ("max_val", C.c_double)]


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


class BinMapper:
    """One feature's value -> bin mapper (BinMapper, bin_mapper.rs:94-135)."""

    def __init__(self, handle):
        self.lib = load_library()
        self.handle = handle
        info = BinMapperInfo()
        self.lib.lgbm_hip_bin_mapper_info(self.handle, C.byref(info))
        for k, _ in BinMapperInfo._fields_:
            setattr(self, k, getattr(info, k))
        self.is_trivial = bool(self.is_trivial)
        ub = np.zeros(self.num_bin, np.float64)
        cats = np.zeros(self.num_bin, np.int32)
        self.lib.lgbm_hip_bin_mapper_bounds(self.handle, ub.ctypes.data_as(C.c_void_p),
                                            cats.ctypes.data_as(C.c_void_p))
        self.bin_type_name = "categorical" if self.bin_type == 1 else "numerical"
        self.upper_bounds = ub if self.bin_type == 0 else None
        self.categories = cats if self.bin_type == 1 else None

    @staticmethod
    def _make(lib, fn, *args):
        h = C.c_void_p()
        rc = fn(*args, C.byref(h))
        if rc != 0:
            buf = C.create_string_buffer(1024)
            lib.lgbm_hip_bin_last_error(buf, C.c_size_t(1024))
            raise HipError(rc, buf.value.decode())
        return BinMapper(h)

    @classmethod
    def from_column(cls, column, forced_upper_bounds=(), **params):
        """BinMapper::find_bin_from_column (bin_mapper.rs:613-651): sample
        min(rows, bin_construct_sample_cnt) rows with data_random_seed, then FindBin."""
        lib = load_library()
        col = _f64(column)
        forced = _f64(forced_upper_bounds)
        p = BinParams.make(**params)
        return cls._make(lib, lib.lgbm_hip_bin_mapper_from_column,
                         col.ctypes.data_as(C.c_void_p), C.c_int64(len(col)), C.byref(p),
                         forced.ctypes.data_as(C.c_void_p), C.c_int32(len(forced)))

    @classmethod
    def from_sample(cls, values, total_sample_cnt=None, categorical=False, min_split_data=0,
                    forced_upper_bounds=(), **params):
        """find_bin_numeric / find_bin_categorical on the given sample values
        (bin_mapper.rs:191-365, 409-560); total_sample_cnt - len(values) zeros implied."""
        lib = load_library()
        v = _f64(values)
        forced = _f64(forced_upper_bounds)
        total = len(v) if total_sample_cnt is None else int(total_sample_cnt)
        p = BinParams.make(**params)
        return cls._make(lib, lib.lgbm_hip_bin_mapper_from_sample,
                         v.ctypes.data_as(C.c_void_p), C.c_int64(len(v)), C.c_int64(total),
                         C.c_int32(int(categorical)), C.byref(p), C.c_int32(min_split_data),
                         forced.ctypes.data_as(C.c_void_p), C.c_int32(len(forced)))

    @classmethod
    def from_sampled_column(cls, sampled, num_rows, **params):
        """find_bin_from_column when the caller has already gathered the column's
        values at sample_indices(num_rows, bin_construct_sample_cnt, data_random_seed)
        (e.g. on the device): the same mapper without the full column on the host."""
        v = _f64(sampled)
        p = dict(DEFAULTS, **params)
        if len(v) != min(num_rows, p["bin_construct_sample_cnt"]):
            raise ValueError("sampled values do not match the sample size")
        filt = (p["min_data_in_leaf"] * len(v)) // num_rows if num_rows else p["min_data_in_leaf"]
        kw = {k: p[k] for k in ("max_bin", "min_data_in_bin", "pre_filter", "use_missing",
                                "zero_as_missing")}
        return cls.from_sample(v, len(v), min_split_data=filt, **kw)

    def value_to_bin(self, values):
        """ValueToBin (bin_mapper.rs:148-189) on the host."""
        v = _f64(values).ravel()
        out = np.zeros(len(v), np.uint32)
        rc = self.lib.lgbm_hip_bin_mapper_value_to_bin(
            self.handle, v.ctypes.data_as(C.c_void_p), C.c_int64(len(v)),
            out.ctypes.data_as(C.c_void_p))
        if rc != 0:
            raise HipError(rc, "value_to_bin")
        return out

    def close(self):
        if self.handle:
            self.lib.lgbm_hip_bin_mapper_free(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sample_indices(num_rows, sample_cnt, seed):
    """Random(seed).Sample(num_rows, min(num_rows, sample_cnt)) (lgbm-core/src/random.rs)."""
    lib = load_library()
    k = max(0, min(num_rows, sample_cnt))
    out = np.zeros(max(k, 1), np.int32)
    n = C.c_int32(0)
    rc = lib.lgbm_hip_sample_indices(C.c_int32(num_rows), C.c_int32(sample_cnt), C.c_int32(seed),
                                     out.ctypes.data_as(C.c_void_p), C.byref(n))
    if rc != 0:
        raise HipError(rc, "sample_indices")
    return out[:n.value].copy()


def feature_mappers(X, categorical_features=(), col_major=False, **params):
    """One mapper per column of X (booster.rs:449-520): categorical columns binned
    whole by find_bin_categorical, the others by find_bin_from_column."""
    X = np.asarray(X)
    cols = X.shape[0] if col_major else X.shape[1]
    cat = set(categorical_features)
    out = []
    for j in range(cols):
        col = X[j] if col_major else X[:, j]
        if j in cat:
            out.append(BinMapper.from_sample(col, len(col), categorical=True,
                                             min_split_data=params.get("min_data_in_leaf", 20),
                                             **{k: v for k, v in params.items()
                                                if k not in ("bin_construct_sample_cnt",
                                                             "data_random_seed")}))
        else:
            out.append(BinMapper.from_column(col, **params))
    return out


def _mapper_array(mappers):
    arr = (C.c_void_p * len(mappers))()
    for i, m in enumerate(mappers):
        arr[i] = m.handle.value if isinstance(m.handle, C.c_void_p) else m.handle
    return arr


def _upload_raw(self, X, mappers, col_major=False):
    """Bin a host matrix on the device into the resident layout
    (lgbm_hip_upload_raw): X float32/float64 [rows, cols] (or [cols, rows] with
    col_major)."""
    X = np.ascontiguousarray(X)
    if X.dtype not in (np.float32, np.float64):
        X = X.astype(np.float64)
    rows, cols = (X.shape[1], X.shape[0]) if col_major else X.shape
    if len(mappers) != cols:
        raise ValueError("one mapper per column")
    self._check(self.lib.lgbm_hip_upload_raw(
        self.ctx, X.ctypes.data_as(C.c_void_p), C.c_int32(1 if X.dtype == np.float64 else 0),
        C.c_int32(int(col_major)), C.c_int64(rows), C.c_int32(cols), _mapper_array(mappers)))
    self.num_data, self.num_features = rows, cols
    self.slot_len = 2 * sum(m.num_bin for m in mappers)


def _upload_raw_device(self, ptr_, dtype, rows, cols, mappers, col_major=False):
    """The same over a device-resident matrix (raw device pointer)."""
    self._check(self.lib.lgbm_hip_upload_raw_device(
        self.ctx, C.c_void_p(ptr_), C.c_int32(1 if np.dtype(dtype) == np.float64 else 0),
        C.c_int32(int(col_major)), C.c_int64(rows), C.c_int32(cols), _mapper_array(mappers)))
    self.num_data, self.num_features = rows, cols
    self.slot_len = 2 * sum(m.num_bin for m in mappers)


def _get_bins(self):
    """The resident bins, feature-major uint8 [features, rows]."""
    out = np.zeros((self.num_features, self.num_data), np.uint8)
    self._check(self.lib.lgbm_hip_get_bins(self.ctx, out.ctypes.data_as(C.c_void_p),
                                           C.c_int64(self.num_data)))
    return out


def _get_bins16(self):
    """The resident bins as uint16 [features, rows] (any bin width)."""
    out = np.zeros((self.num_features, self.num_data), np.uint16)
    self._check(self.lib.lgbm_hip_get_bins16(self.ctx, out.ctypes.data_as(C.c_void_p),
                                             C.c_int64(self.num_data)))
    return out


HipBackend.get_bins16 = _get_bins16
HipBackend.upload_raw = _upload_raw
HipBackend.upload_raw_device = _upload_raw_device
HipBackend.get_bins = _get_bins

__all__ = ["BinMapper", "BinParams", "feature_mappers", "sample_indices", "DEFAULTS"]
