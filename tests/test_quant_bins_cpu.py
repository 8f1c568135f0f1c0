"""num_grad_quant_bins other than 2 and 4, pinned on the reference's quantized goldens
(crates/oracle-harness/tests/quantized_parity.rs; fixture copied by
tests/golden/make_quantized_golden.py): real LightGBM 4.6 trained on the 512 x 6
corpus with use_quantized_grad, num_grad_quant_bins 128 and deterministic rounding, with
and without quantization and with quant_train_renew_leaf.  The reference gates its own
learner against them with these bounds (quantized_parity.rs:126-153,196-203): the
exact model within 1e-5, the quantized one within 1e-2, and the quantization and
renewal effects in C++'s regime.  The oracle (the reference's CPU path restated) is
held to the same gates, then the discretizer at 128 bins is checked by hand."""
import json
import os

import numpy as np

from lightgbm_rs_amd import GainConfig, feature_mappers, feature_meta
from oracle import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "quantized")


def _train(X, y, p, quantized, renew=False):
    ms = feature_mappers(X, max_bin=p["max_bin"], min_data_in_leaf=p["min_data_in_leaf"])
    bins = np.stack([m.value_to_bin(X[:, j]) for j, m in enumerate(ms)]).astype(np.uint8)
    meta = [feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f)
            for f, m in enumerate(ms)]
    ub = np.concatenate([m.upper_bounds for m in ms])
    cfg = GainConfig.make(min_data_in_leaf=p["min_data_in_leaf"])
    scores, _ = oracle.train(bins, meta, ub, y, cfg, oracle.OBJECTIVE_BINARY, p["num_leaves"], -1,
                             10, p["learning_rate"], quantized=quantized,
                             quant_bins=p["num_grad_quant_bins"], stochastic=False,
                             quant_renew_leaf=renew)
    return 1.0 / (1.0 + np.exp(-scores))


def _delta(a, b):
    d = np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))
    return d.max(), d.mean()


def test_oracle_128_bins_in_the_reference_gates():
    z = np.load(os.path.join(GOLD, "quant_binary.npz"))
    p = json.loads(str(z["params"]))["params"]
    assert p["num_grad_quant_bins"] == 128 and not p["stochastic_rounding"]
    X, y = z["X"], z["y"]
    exact = _train(X, y, p, False)
    quant = _train(X, y, p, True)
    renew = _train(X, y, p, True, renew=True)
    xe_max, _ = _delta(exact, z["pred_exact"])
    qe_max, _ = _delta(quant, z["pred"])
    assert xe_max < 1e-5, xe_max
    assert qe_max < 1e-2, qe_max
    rq_max, rq_mean = _delta(quant, exact)
    cq_max, cq_mean = _delta(z["pred"], z["pred_exact"])
    assert rq_max > 1e-6, "quantization had no effect"
    assert rq_mean < 2.0 * max(cq_mean, 1e-4) and rq_max < 3.0 * max(cq_max, 1e-3)
    re_max, re_mean = _delta(renew, quant)
    ce_max, ce_mean = _delta(z["pred_renew"], z["pred"])
    assert re_max > 1e-6, "renewal had no effect"
    assert re_mean < 5.0 * max(ce_mean, 1e-4) and re_max < 5.0 * max(ce_max, 1e-3)


def test_discretizer_128_bins_by_hand():
    """gradient_discretizer.rs:145-188 at 128 bins, deterministic: grad scale max|g| /
    (128 / 2), hess scale max|h| / 128, q = trunc(x / scale +- 0.5) saturated to i8 (a
    hessian at its maximum gives q = 128 -> 127), values f32(q * scale)."""
    g = np.array([0.5, -0.25, 0.1, -0.5, 0.003, 0.0], np.float32)
    h = np.array([0.25, 0.0625, 0.2, 0.25, 0.01, 0.125], np.float32)
    dg, dh, disc, scales = oracle.quantize(g, h, bins=128, stochastic=False)
    gs, hs = 0.5 / 64, 0.25 / 128
    assert scales[0] == gs and scales[1] == hs
    qg = [int(np.trunc(float(v) / gs + (0.5 if v >= 0 else -0.5))) for v in g]
    qh = [min(int(np.trunc(float(v) / hs + 0.5)), 127) for v in h]
    assert qh[0] == 127 and qh[3] == 127  # 128 saturates
    assert disc[1::2].tolist() == qg and disc[0::2].tolist() == qh
    assert np.array_equal(dg, np.array([np.float32(q * gs) for q in qg], np.float32))
    assert np.array_equal(dh, np.array([np.float32(q * hs) for q in qh], np.float32))
