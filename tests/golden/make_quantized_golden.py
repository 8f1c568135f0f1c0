"""Copy the reference's quantized-training goldens into a compact fixture.

Run in the build container (where /root/reference exists):

    python tests/golden/make_quantized_golden.py

Sources (data files of the reference's own test, quantized_parity.rs):

  crates/oracle-harness/tests/fixtures/quantized/quant_binary.xy.csv   (512 rows x 6
      features + label, the training table)
  .../quant_binary.pred          C++ LightGBM 4.6 predictions, use_quantized_grad with
                                 num_grad_quant_bins 128, deterministic rounding
  .../quant_binary.pred_exact    the same without quantization
  .../quant_binary.pred_renew    quantized with quant_train_renew_leaf
  .../quant_binary.json          the parameters (the model text is not kept)

Output: tests/golden/quantized/quant_binary.npz with X (float64 [512, 6]), y (float32),
pred, pred_exact, pred_renew (float64 [512]) and the parameters as a JSON string.
"""
import json
import os

import numpy as np

SRC = "/root/reference/crates/oracle-harness/tests/fixtures/quantized"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quantized")


def preds(name):
    with open(os.path.join(SRC, name)) as f:
        return np.array([float(l) for l in f if l.strip()], dtype=np.float64)


def main():
    rows = []
    with open(os.path.join(SRC, "quant_binary.xy.csv")) as f:
        for line in f:
            if line.startswith("#") or not line.strip():
                continue
            rows.append([float(v) for v in line.split(",")])
    a = np.array(rows, dtype=np.float64)
    with open(os.path.join(SRC, "quant_binary.json")) as f:
        meta = json.load(f)
    params = {k: meta[k] for k in ("lightgbm_version", "params", "num_round", "n", "num_features")}
    os.makedirs(OUT, exist_ok=True)
    np.savez_compressed(os.path.join(OUT, "quant_binary.npz"), X=a[:, :-1],
                        y=a[:, -1].astype(np.float32), pred=preds("quant_binary.pred"),
                        pred_exact=preds("quant_binary.pred_exact"),
                        pred_renew=preds("quant_binary.pred_renew"), params=json.dumps(params))


if __name__ == "__main__":
    main()
