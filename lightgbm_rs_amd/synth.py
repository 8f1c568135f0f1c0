"""Synthetic inputs of BASELINE.json's configurations (no datasets offline).

config0_like(): configs[0] — N rows x 28 float32 features ~N(0,1), the same logistic
label, binned to <= 255 quantile bins (the f32-gradient CPU-reference case).

config3_raw_host() / config3_binned(): configs[3] — N rows x 100 float32 features (80
~N(0,1), 20 integer-coded categoricals with 32 levels), class = argmax of 10 random
linear projections of the features (the categoricals one-hot encoded) + Gumbel noise;
numerical features binned like
configs[1] (max_bin 255), categorical ones by find_bin_categorical over the whole
column (booster.rs:449-520).

config1_like(): configs[1] — N rows x 28 float32 features (21 ~N(0,1), 7 derived as
products / abs of pairs), logistic label logit = w.x + 0.5*x0*x1 + N(0, 0.1) with
w ~ N(0,1), binned to <= max_bin bins per feature (u8) by this library's BinMapper
(BinMapper::find_bin_from_column on a bin_construct_sample_cnt = 200000 row sample,
then ValueToBin), so the feature descriptors are the reference's: most_freq_bin,
default_bin, missing type and the offset rule come from the mappers.  With `device`
set to a torch CUDA device the generation and a quantile binning run there (same
recipe, torch's generator).
"""
import os

import numpy as np

from ._abi import FeatureMeta

DERIVED = [("mul", 0, 1), ("mul", 2, 3), ("abs", 4, None), ("mul", 5, 6), ("absmul", 7, 8),
           ("mul", 9, 10), ("abs", 11, None)]


def _meta_for(num_bins):
    meta = []
    for f, nb in enumerate(num_bins):
        m = FeatureMeta()
        m.num_bin = nb
        m.offset = 1
        m.min_bin = 0
        m.max_bin = nb - 1
        m.default_bin = nb
        m.most_freq_bin = 0
        m.missing_type = 0
        m.real_feature_index = f
        meta.append(m)
    return meta


def _derive(X, lib):
    out = []
    for kind, a, b in DERIVED:
        if kind == "mul":
            out.append(X[a] * X[b])
        elif kind == "abs":
            out.append(lib.abs(X[a]))
        else:
            out.append(lib.abs(X[a] * X[b]))
    return out


def config0_like(n, seed=0x5EED0000, max_bin=255):
    return config1_like(n, seed=seed, max_bin=max_bin, derived=False)


def config1_raw_host(n, seed=0x5EED0001, derived=True):
    """configs[1]'s raw table on the host: X float32 [28, n] (one feature per row) and
    the labels, drawn with numpy's generator."""
    rng = np.random.default_rng(seed)
    if derived:
        X = rng.standard_normal((21, n), dtype=np.float32)
        X = np.concatenate([X, np.stack(_derive(X, np))], axis=0)
    else:
        X = rng.standard_normal((28, n), dtype=np.float32)
    w = rng.standard_normal(28).astype(np.float32)
    logit = w @ X + 0.5 * X[0] * X[1] + rng.normal(0, 0.1, n).astype(np.float32)
    y = (rng.random(n, dtype=np.float32) < 1.0 / (1.0 + np.exp(-logit))).astype(np.float32)
    return X, y


def config1_like(n, seed=0x5EED0001, max_bin=63, device=None, derived=True):
    if device is not None:
        return _config1_torch(n, seed, max_bin, device)
    X, y = config1_raw_host(n, seed, derived)
    bins, meta, upper = bin_with_mappers(X, max_bin)
    return bins, meta, upper, y


def bin_with_mappers(X, max_bin, min_data_in_leaf=20):
    """X [F, n] -> (bins u8 [F, n], feature meta, concatenated upper bounds) with this
    library's BinMapper: find_bin_from_column's 200000-row sample (data_random_seed 1),
    ValueToBin on the host, the descriptors of the booster's feature columns
    (booster.rs:449-520)."""
    from .backend import feature_meta
    from .binning import BinMapper, sample_indices
    F, n = X.shape
    idx = sample_indices(n, 200000, 1)
    bins = np.zeros((F, n), dtype=np.uint8)
    meta, upper = [], []
    for f in range(F):
        m = BinMapper.from_sampled_column(X[f, idx].astype(np.float64), n, max_bin=max_bin,
                                          min_data_in_leaf=min_data_in_leaf)
        bins[f] = m.value_to_bin(X[f]).astype(np.uint8)
        meta.append(feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f))
        upper.extend(m.upper_bounds.tolist())
    return bins, meta, np.array(upper, dtype=np.float64)


def config1_raw(n, seed=0x5EED0001, device=None):
    """configs[1]'s raw table before binning: X as a torch float32 tensor [28, n] on
    `device` (column-major: one feature per row) and the labels as numpy float32.
    The same recipe and generator draws as config1_like(device=...)."""
    import torch

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    X = torch.randn((21, n), generator=gen, device=device, dtype=torch.float32)
    X = torch.cat([X, torch.stack(_derive(X, torch))], dim=0)
    w = torch.randn(28, generator=gen, device=device, dtype=torch.float32)
    noise = torch.randn(n, generator=gen, device=device, dtype=torch.float32) * 0.1
    logit = w @ X + 0.5 * X[0] * X[1] + noise
    u = torch.rand(n, generator=gen, device=device, dtype=torch.float32)
    y = (u < torch.sigmoid(logit)).to(torch.float32)
    return X.contiguous(), y.cpu().numpy()


def _config1_torch(n, seed, max_bin, device):
    import torch

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    X = torch.randn((21, n), generator=gen, device=device, dtype=torch.float32)
    X = torch.cat([X, torch.stack(_derive(X, torch))], dim=0)
    w = torch.randn(28, generator=gen, device=device, dtype=torch.float32)
    noise = torch.randn(n, generator=gen, device=device, dtype=torch.float32) * 0.1
    logit = w @ X + 0.5 * X[0] * X[1] + noise
    u = torch.rand(n, generator=gen, device=device, dtype=torch.float32)
    y = (u < torch.sigmoid(logit)).to(torch.float32)
    step = max(1, n // 200000)
    qgrid = torch.linspace(0, 1, max_bin + 1, device=device, dtype=torch.float32)[1:-1]
    bins = torch.empty((28, n), dtype=torch.uint8, device=device)
    upper, nbs = [], []
    for f in range(28):
        qs = torch.unique(torch.quantile(X[f, ::step].contiguous(), qgrid))
        bins[f] = torch.bucketize(X[f], qs, right=False).to(torch.uint8)
        nbs.append(int(qs.numel()) + 1)
        upper.extend([float(q) for q in qs.cpu()] + [float("inf")])
    return (bins.cpu().numpy(), _meta_for(nbs), np.array(upper, dtype=np.float64),
            y.cpu().numpy())


def config3_raw_host(n, seed=0x5EED0003, num_class=10, n_num=80, n_cat=20, levels=32):
    """configs[3]'s raw table on the host: X float32 [n_num + n_cat, n] (one feature per
    row; the last n_cat rows hold category codes 0..levels-1), the class labels as
    float32, and the categorical feature positions."""
    rng = np.random.default_rng(seed)
    F = n_num + n_cat
    X = np.empty((F, n), dtype=np.float32)
    X[:n_num] = rng.standard_normal((n_num, n), dtype=np.float32)
    X[n_num:] = rng.integers(0, levels, (n_cat, n)).astype(np.float32)
    # the projections read the numerical features directly and each categorical one
    # through its one-hot encoding (a random weight per (class, level))
    W = rng.standard_normal((num_class, n_num)).astype(np.float32) / np.float32(np.sqrt(n_num))
    E = rng.standard_normal((n_cat, levels, num_class)).astype(np.float32) * np.float32(0.5)
    logits = W @ X[:n_num]
    for j in range(n_cat):
        logits += E[j][X[n_num + j].astype(np.int64)].T
    u = rng.random((num_class, n), dtype=np.float32)
    gumbel = -np.log(-np.log(np.clip(u, 1e-12, 1.0 - 1e-7)))
    y = np.argmax(logits + gumbel, axis=0).astype(np.float32)
    return X, y, list(range(n_num, F))


def config3_mappers(X, cat, max_bin=255, min_data_in_leaf=20):
    """configs[3]'s mappers for X [F, n]: categorical features binned whole
    (find_bin_categorical), numerical ones from find_bin_from_column's 200000-row
    sample.  Returns (mappers, feature meta, per-bin values: numerical upper bounds,
    categorical category codes)."""
    from .backend import feature_meta
    from .binning import BinMapper, sample_indices
    F, n = X.shape
    idx = sample_indices(n, 200000, 1)
    meta, vals, mappers = [], [], []
    for f in range(F):
        if f in cat:
            m = BinMapper.from_sample(X[f].astype(np.float64), n, categorical=True,
                                      min_split_data=min_data_in_leaf, max_bin=max_bin)
            vals.extend(float(c) for c in m.categories)
        else:
            m = BinMapper.from_sampled_column(X[f, idx].astype(np.float64), n, max_bin=max_bin,
                                              min_data_in_leaf=min_data_in_leaf)
            vals.extend(m.upper_bounds.tolist())
        meta.append(feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f,
                                 bin_type=m.bin_type))
        mappers.append(m)
    return mappers, meta, np.array(vals, dtype=np.float64)


def config3_binned(n, seed=0x5EED0003, max_bin=255, min_data_in_leaf=20, **kw):
    """configs[3] binned: (bins u8 [F, n], feature meta, per-bin values (numerical upper
    bounds, categorical category codes), labels, categorical positions, raw X)."""
    X, y, cat = config3_raw_host(n, seed, **kw)
    mappers, meta, vals = config3_mappers(X, cat, max_bin, min_data_in_leaf)
    bins = np.zeros(X.shape, dtype=np.uint8)
    for f, m in enumerate(mappers):
        bins[f] = m.value_to_bin(X[f]).astype(np.uint8)
    return bins, meta, vals, y, cat, X, mappers


def _bin_columns(X, max_bin, min_data_in_leaf=20):
    """X [F, n] -> (bins u8 [F, n], feature meta, concatenated upper bounds, mappers)
    with this library's BinMapper (find_bin_from_column's 200000-row sample)."""
    from .backend import feature_meta
    from .binning import BinMapper, sample_indices
    F, n = X.shape
    idx = sample_indices(n, 200000, 1)
    bins = np.zeros((F, n), dtype=np.uint8)
    meta, upper, mappers = [], [], []
    for f in range(F):
        m = BinMapper.from_sampled_column(X[f, idx].astype(np.float64), n, max_bin=max_bin,
                                          min_data_in_leaf=min_data_in_leaf)
        bins[f] = m.value_to_bin(X[f]).astype(np.uint8)
        meta.append(feature_meta(m.num_bin, m.most_freq_bin, m.missing_type, m.default_bin, f))
        upper.extend(m.upper_bounds.tolist())
        mappers.append(m)
    return bins, meta, np.array(upper, dtype=np.float64), mappers


def config2_raw_host(n, seed=0x5EED0002, F=2000, informative=50):
    """configs[2]'s raw table: X float32 [F, n] with 90% exact zeros per feature and
    LogNormal(0, 1) nonzeros; the L2 target = sum over `informative` random features of
    x * U(-1, 1) + N(0, 0.5)."""
    rng = np.random.default_rng(seed)
    X = np.zeros((F, n), dtype=np.float32)
    for f0 in range(0, F, 64):  # 64 features per draw
        blk = X[f0:f0 + 64]
        nz = rng.random(blk.shape, dtype=np.float32) < 0.1
        blk[nz] = np.exp(rng.standard_normal(int(nz.sum()), dtype=np.float32))
    feats = rng.choice(F, size=informative, replace=False)
    w = rng.uniform(-1.0, 1.0, informative)
    y = (X[feats].astype(np.float64).T @ w + rng.normal(0.0, 0.5, n)).astype(np.float32)
    return X, y


def config2_binned(n, seed=0x5EED0002, F=2000, max_bin=255):
    X, y = config2_raw_host(n, seed, F)
    bins, meta, upper, _ = _bin_columns(X, max_bin)
    return bins, meta, upper, y


def sample_mappers(X, max_bin, min_data_in_leaf=20):
    """One BinMapper per feature row of X [F, n] from find_bin_from_column's
    200000-row sample (data_random_seed 1): the mappers lgbm_hip_upload_raw bins with."""
    from concurrent.futures import ThreadPoolExecutor
    from .binning import BinMapper, sample_indices
    F, n = X.shape
    idx = sample_indices(n, 200000, 1)

    def one(f):  # the C++ mapper construction runs without the GIL
        return BinMapper.from_sampled_column(X[f, idx].astype(np.float64), n, max_bin=max_bin,
                                             min_data_in_leaf=min_data_in_leaf)
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        return list(ex.map(one, range(F)))


def config4_raw_host(n, seed=0x5EED0004, F=700, mean_group=120):
    """configs[4]'s raw table: X float32 [F, n] ~U(0, 1) with 30% zeros, query groups of
    Poisson(mean_group) sizes (at least 1; the last one cut at n), graded relevance 0-4
    from the quintiles of a random linear score plus noise.  Returns (X, relevance
    float32, group sizes int32)."""
    rng = np.random.default_rng(seed)
    X = rng.random((F, n), dtype=np.float32)
    for f0 in range(0, F, 64):  # 30% zeros, 64 features per draw
        blk = X[f0:f0 + 64]
        blk[rng.random(blk.shape, dtype=np.float32) < 0.3] = 0.0
    w = rng.standard_normal(F)
    s = X.astype(np.float64).T @ w
    s += rng.normal(0.0, float(np.std(s)) * 0.5 + 1e-12, n)
    y = np.searchsorted(np.quantile(s, [0.2, 0.4, 0.6, 0.8]), s, side="right").astype(np.float32)
    sizes = []
    left = n
    while left > 0:
        k = max(1, int(rng.poisson(mean_group)))
        k = min(k, left)
        sizes.append(k)
        left -= k
    return X, y, np.array(sizes, dtype=np.int32)


def config4_binned(n, seed=0x5EED0004, F=700, max_bin=255):
    X, y, groups = config4_raw_host(n, seed, F)
    bins, meta, upper, _ = _bin_columns(X, max_bin)
    return bins, meta, upper, y, groups
