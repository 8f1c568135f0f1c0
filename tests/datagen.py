"""Seeded synthetic inputs shared by the parity tests and bench.py.

Binned columns are generated directly (the binning step sits before the path):
each feature gets a num_bin, a most-frequent bin (0 -> offset 1, else FixHistogram
is active), a missing type and matching bin_upper_bound values.
"""
import numpy as np

from lightgbm_rs_amd._abi import FeatureMeta


def make_binned(n, F, seed, max_bin=64, missing_mix=True, mfb_mix=True):
    rng = np.random.default_rng(seed)
    bins = np.zeros((F, n), dtype=np.uint8)
    meta, upper = [], []
    for f in range(F):
        nb = int(rng.integers(2, max_bin + 1)) if f % 7 else max_bin
        # skewed bin distribution (a realistic most-frequent bin)
        p = rng.dirichlet(np.full(nb, 0.7))
        col = rng.choice(nb, size=n, p=p).astype(np.uint8)
        bins[f] = col
        counts = np.bincount(col, minlength=nb)
        mfb = int(np.argmax(counts)) if (mfb_mix and f % 3 == 1) else 0
        mt = 0
        if missing_mix and nb > 2:
            mt = [0, 0, 1, 2][f % 4]
        m = FeatureMeta()
        m.num_bin = nb
        m.offset = 1 if mfb == 0 else 0
        m.min_bin = 0
        m.max_bin = nb - 1
        m.default_bin = mfb if mt == 1 else (nb if mt == 0 else 0)
        m.most_freq_bin = mfb
        m.missing_type = mt
        m.real_feature_index = f
        meta.append(m)
        upper.extend((np.arange(nb) + 0.5).tolist())
    return bins, meta, np.array(upper, dtype=np.float64)


def binary_gh(n, seed):
    """Gradients/hessians shaped like binary logloss at a random score."""
    rng = np.random.default_rng(seed + 1000)
    s = rng.normal(0.0, 1.5, size=n)
    y = rng.random(n) < 1.0 / (1.0 + np.exp(-s))
    p = 1.0 / (1.0 + np.exp(-s))
    g = (p - y).astype(np.float32)
    h = (p * (1.0 - p)).astype(np.float32)
    return g, h, y.astype(np.float32)


from lightgbm_rs_amd.synth import config1_like  # noqa: E402,F401
