"""Extract the reference's committed prediction goldens into compact fixtures.

Run in the build container (where /root/reference exists):

    python tests/golden/make_predict_golden.py

Sources (data files of the reference's own tests):

  crates/lgbm-model/tests/fixtures/models/<corpus>/model.txt      (LightGBM v4 model text)
  crates/lgbm-model/tests/fixtures/models/<corpus>/raw.txt        (per row: f64 bits of the raw scores)
  crates/lgbm-model/tests/fixtures/models/<corpus>/transformed.txt  (per row: f64 bits, ConvertOutput)
  crates/lgbm-model/tests/fixtures/models/<corpus>/leaf.txt       (per row: leaf id of every tree)
  crates/lgbm-dataset/tests/fixtures/examples/{binary,regression}.train  (the input table)

The corpus -> input table map is the reference tests' (predict_leaf_parity.rs:27-32):
binary and categorical use binary.train, regression and multiclass regression.train.
The categorical corpus was trained and predicted on binary.train with columns 0, 5,
10 and 15 integerized as mod(round(|3x|), 5) (xtask/py/model_capture.py:254-262); the
same transform is applied here.
The subrange corpus adds subrange.txt: raw scores of iteration slices (start, num).
Only the first ROWS rows are kept.  Output: tests/golden/predict/<corpus>_model.txt
(the model text, unchanged) and <corpus>.npz with X (float32 [rows, cols]), raw and
transformed (float64 [rows, outputs]), leaf (int32 [rows, trees]) and, for subrange,
slice_start / slice_num / slice_raw (float64 [slices, rows]).
"""
import os

import numpy as np

REF = "/root/reference/crates"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "predict")
ROWS = 1000
CORPORA = {"binary": "binary.train", "categorical": "binary.train",
           "regression": "regression.train", "multiclass": "regression.train",
           "subrange": "regression.train"}


def load_table(path, rows, categorical=False):
    X = []
    with open(path) as f:
        for line in f:
            line = line.strip()
            if not line:
                continue
            X.append([float(t) for t in line.split()[1:]])
            if len(X) == rows:
                break
    X = np.array(X, dtype=np.float64)
    if categorical:
        for j in (0, 5, 10, 15):
            X[:, j] = np.mod(np.round(np.abs(X[:, j] * 3.0)), 5.0)
    return X.astype(np.float32)


def load_rows(path, rows, dtype):
    out = []
    with open(path) as f:
        for line in f:
            line = line.strip()
            if not line or line.startswith("#"):
                continue
            out.append([int(t) for t in line.split(";") if t])
            if len(out) == rows:
                break
    a = np.array(out, dtype=np.uint64 if dtype == "f64" else np.int64)
    return a.view(np.float64) if dtype == "f64" else a.astype(np.int32)


def load_slices(path, rows):
    """subrange.txt: `SLICE start=<s> num=<n>` headers, each followed by one line of
    f64 bits for every row (predict_subrange.rs:36-70)."""
    starts, nums, vals = [], [], []
    with open(path) as f:
        lines = [l.strip() for l in f if l.strip()]
    for h, data in zip(lines[0::2], lines[1::2]):
        kv = dict(t.split("=") for t in h.split()[1:])
        starts.append(int(kv["start"]))
        nums.append(int(kv["num"]))
        vals.append([int(t) for t in data.split(";") if t][:rows])
    return (np.array(starts, np.int32), np.array(nums, np.int32),
            np.array(vals, np.uint64).view(np.float64))


def main():
    os.makedirs(OUT, exist_ok=True)
    for corpus, table in CORPORA.items():
        d = os.path.join(REF, "lgbm-model/tests/fixtures/models", corpus)
        X = load_table(os.path.join(REF, "lgbm-dataset/tests/fixtures/examples", table), ROWS,
                       categorical=corpus == "categorical")
        raw = load_rows(os.path.join(d, "raw.txt"), ROWS, "f64")
        tr = load_rows(os.path.join(d, "transformed.txt"), ROWS, "f64")
        leaf = load_rows(os.path.join(d, "leaf.txt"), ROWS, "i32")
        with open(os.path.join(d, "model.txt"), "rb") as f:
            text = f.read()
        with open(os.path.join(OUT, corpus + "_model.txt"), "wb") as f:
            f.write(text)
        extra = {}
        if corpus == "subrange":
            st, nm, sv = load_slices(os.path.join(d, "subrange.txt"), ROWS)
            extra = {"slice_start": st, "slice_num": nm, "slice_raw": sv}
        np.savez_compressed(os.path.join(OUT, corpus + ".npz"), X=X, raw=raw, transformed=tr,
                            leaf=leaf, **extra)
        print(corpus, X.shape, raw.shape, tr.shape, leaf.shape)


if __name__ == "__main__":
    main()
