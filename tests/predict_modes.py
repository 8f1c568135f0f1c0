"""Readers for the reference's prediction-mode captures (tests/golden/predict_modes/)."""
import os

import numpy as np

DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "predict_modes")


def _bits(tokens):
    return np.array([int(t) for t in tokens], dtype=np.uint64).view(np.float64)


def corpus(name):
    """(model text, X float32 [rows, cols], cells [(freq, margin, raw [rows, width])])."""
    d = os.path.join(DIR, name)
    text = open(os.path.join(d, "model.txt")).read()
    rows = [line.split() for line in open(os.path.join(d, "X.txt"))
            if line.strip() and not line.startswith("#")]
    X = np.stack([_bits(r) for r in rows]).astype(np.float32)
    cells, cur = [], None
    for line in open(os.path.join(d, "early_stop.txt")):
        toks = line.split()
        if not toks or toks[0].startswith("#"):
            continue
        if toks[0] == "CELL":
            kv = dict(t.split("=") for t in toks[1:])
            cur = (int(kv["freq"]), float(kv["margin"]), [])
            cells.append(cur)
        else:
            cur[2].append(_bits(toks))
    return text, X, [(f, m, np.stack(r)) for f, m, r in cells]


def contrib(name):
    """(model text, X float32 [rows, cols], contributions f64 [rows, width]) of the real
    binary's `predict(pred_contrib=True)` capture."""
    d = os.path.join(DIR, name)
    text = open(os.path.join(d, "model.txt")).read()
    rows = [line.split() for line in open(os.path.join(d, "X.txt"))
            if line.strip() and not line.startswith("#")]
    X = np.stack([_bits(r) for r in rows]).astype(np.float32)
    out = [_bits(line.split()) for line in open(os.path.join(d, "contrib.txt"))
           if line.strip() and not line.startswith("#")]
    return text, X, np.stack(out)
