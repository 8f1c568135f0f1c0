"""Readers for the reference's binning goldens (tests/golden/binning/*.txt.gz).

Record forms: `CASE|MCASE|CCASE|DATASET k=v ...` headers, `VALUES`/`MATRIX` f64 bit
patterns separated by ';', `GOLDEN|MAPPER|FEATURE k=v ...` expected mapper fields
(`upper=` as f64 bits), `ASSIGN [f=<i>] a;b;...` per-row bins, `C2B cat:bin;...`
and `B2C cat;...` for categorical folds."""
import gzip
import os

import numpy as np

DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "binning")


def bits_to_f64(s):
    toks = [t for t in s.split(";") if t]
    return np.array([int(t) for t in toks], dtype=np.uint64).view(np.float64)


def ints(s):
    return np.array([int(t) for t in s.split(";") if t], dtype=np.int64)


def kv(tokens):
    return dict(t.split("=", 1) for t in tokens if "=" in t)


def lines(name):
    with gzip.open(os.path.join(DIR, name + ".txt.gz"), "rt") as f:
        return f.read().splitlines()


def cases(name):
    """Flat case records of numeric_binning / missing_edge_cases / categorical_folding."""
    out, cur = [], None
    for line in lines(name):
        head, _, rest = line.partition(" ")
        if head in ("CASE", "MCASE", "CCASE"):
            cur = {"params": kv(rest.split())}
            out.append(cur)
        elif cur is None:
            continue
        elif head == "VALUES":
            cur["values"] = bits_to_f64(rest)
        elif head in ("GOLDEN", "MAPPER"):
            cur["mapper"] = kv(rest.split())
        elif head == "ASSIGN":
            cur["assign"] = ints(rest).astype(np.uint32)
        elif head == "C2B":
            cur["c2b"] = {int(a): int(b) for a, b in (t.split(":") for t in rest.split(";") if t)}
        elif head == "B2C":
            cur["b2c"] = ints(rest).astype(np.int32)
    return out


def datasets(name):
    """DATASET records (example_dataset_binning / default_config_ingest): params,
    optional matrix [rows, cols] f64, and per-feature mapper fields + assign."""
    out, cur = [], None
    for line in lines(name):
        head, _, rest = line.partition(" ")
        if head == "DATASET":
            cur = {"params": kv(rest.split()), "features": {}, "assign": {}}
            out.append(cur)
        elif cur is None:
            continue
        elif head == "MATRIX":
            toks = rest.split(" ", 2)
            p = kv(toks[:2])
            cur["matrix"] = bits_to_f64(toks[2]).reshape(int(p["rows"]), int(p["cols"]))
        elif head == "FEATURE":
            p = kv(rest.split())
            cur["features"][int(p["f"])] = p
        elif head == "ASSIGN":
            f, _, vals = rest.partition(" ")
            cur["assign"][int(f.split("=")[1])] = ints(vals).astype(np.uint32)
    return out


def examples():
    with np.load(os.path.join(DIR, "examples.npz")) as z:
        return {k: z[k] for k in z.files}
