"""MI355X-native (gfx950) GBDT tree-learner hot path for lightgbm_rs.

The compute lives in liblgbm_hip.so (HIP kernels + C-ABI, include/lgbm_hip.h);
this package is the Python host mirror of the reference's `Backend` seam.
"""
from ._abi import FeatureMeta, GainConfig, SplitInfo, BatchedFeature  # noqa: F401
from .backend import (HipBackend, HipError, Model, binary_boost_from_score, boost_from_score,  # noqa: F401,E501
                      feature_meta, load_library)
from .binning import BinMapper, feature_mappers, sample_indices  # noqa: F401
