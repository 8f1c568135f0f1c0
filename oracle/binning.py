"""CPU restatement of ValueToBin for checking the device binning kernel.

Test infrastructure only (tests/ and the benchmark's CPU baseline use it; the
product never does).  Follows BinMapper::value_to_bin
(crates/lgbm-dataset/src/bin_mapper.rs:148-189), written as a vectorised search
instead of the reference's bisection:

  numerical: NaN -> the NaN bin (num_bin - 1) when missing_type is NaN, else the
             value 0.0; then the first bin b in [0, last] with value <= upper[b]
             (last = num_bin - 1, minus one more with a NaN bin), or `last`;
  categorical: NaN or a negative int(value) -> 0; a known category -> its bin;
             an unknown one -> 0.

Pinned by the reference's ASSIGN vectors (numeric_binning.txt, missing_edge_cases.txt,
categorical_folding.txt, example_dataset_binning.txt) in tests/test_binning_cpu.py.
"""
import numpy as np

MISSING_NAN = 2


def value_to_bin_numeric(values, upper, missing_type):
    v = np.asarray(values, dtype=np.float64)
    upper = np.asarray(upper, dtype=np.float64)
    nb = len(upper)
    nan_bin = missing_type == MISSING_NAN
    last = nb - 1 - (1 if nan_bin else 0)
    isnan = np.isnan(v)
    w = np.where(isnan, 0.0, v)
    out = np.minimum(np.searchsorted(upper[:last + 1], w, side="left"), last).astype(np.uint32)
    if nan_bin:
        out[isnan] = nb - 1
    return out


def value_to_bin_categorical(values, categories):
    """categories[b] = the category of bin b (bin 0: -1)."""
    v = np.asarray(values, dtype=np.float64)
    lut = {int(c): b for b, c in enumerate(categories) if b > 0}
    out = np.zeros(len(v), np.uint32)
    for i, x in enumerate(v):
        if np.isnan(x):
            continue
        k = int(max(min(x, 2147483647.0), -2147483648.0))
        if k >= 0:
            out[i] = lut.get(k, 0)
    return out
