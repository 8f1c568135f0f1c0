"""Copy the reference's committed binning goldens (gzip-compressed, unchanged text).

Run in the build container (where /root/reference exists):

    python tests/golden/make_binning_golden.py

Sources (data files of the reference's own tests, crates/lgbm-dataset/tests/fixtures/):

  numeric_binning.txt          45 numeric FindBin + ValueToBin cases (CASE / VALUES /
                               GOLDEN / ASSIGN; values and bounds as f64 bit patterns)
  missing_edge_cases.txt       missing-value routing across use_missing / zero_as_missing
  categorical_folding.txt      categorical FindBin folds (C2B / B2C maps) + ValueToBin
  example_dataset_binning.txt  FindBin + ValueToBin over LightGBM's example datasets
  default_config_ingest.txt    the scaled pre-filter path (feature_pre_filter=true,
                               bin_construct_sample_cnt < num_rows) with its raw matrix

and, for example_dataset_binning.txt, the input it was captured on: the first 500
rows of examples/{regression,binary}.train (label column dropped, values parsed as
f64 the way example_dataset_parity.rs:148-180 reads them), saved as
examples.npz {regression, binary} float64 [500, 28].
"""
import gzip
import os
import shutil

import numpy as np

FIX = "/root/reference/crates/lgbm-dataset/tests/fixtures"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "binning")
FILES = ["numeric_binning.txt", "missing_edge_cases.txt", "categorical_folding.txt",
         "example_dataset_binning.txt", "default_config_ingest.txt"]


def main():
    os.makedirs(OUT, exist_ok=True)
    for name in FILES:
        with open(os.path.join(FIX, name), "rb") as src, \
                gzip.GzipFile(os.path.join(OUT, name + ".gz"), "wb", mtime=0) as dst:
            shutil.copyfileobj(src, dst)
        print(name)
    tables = {}
    for name in ("regression", "binary"):
        rows = []
        with open(os.path.join(FIX, "examples", name + ".train")) as f:
            for line in f:
                vals = line.split()
                if vals:
                    rows.append([float(t) for t in vals[1:]])
                if len(rows) == 500:
                    break
        tables[name] = np.array(rows, dtype=np.float64)
    np.savez_compressed(os.path.join(OUT, "examples.npz"), **tables)


if __name__ == "__main__":
    main()
