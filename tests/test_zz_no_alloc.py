"""lgbm_hip_find_best_splits_noalloc (no allocation: its working memory is the
library's fixed per-device array) against lgbm_hip_find_best_splits on the same
inputs, through the C-ABI with device buffers: bit-exact SplitInfo on two calls in a
row (the second with fewer features and a shorter histogram, so stale working memory
from the first would show), plus its size limit and its refusal of invalid features
with the host entry's status codes."""
import ctypes as C

import numpy as np
import pytest

from lightgbm_rs_amd import GainConfig, HipBackend
from lightgbm_rs_amd._abi import BatchedFeature, SplitInfo

pytestmark = pytest.mark.gpu
MAX_FEATS = 8192  # LGBM_HIP_NOALLOC_MAX_FEATURES


class Dev:
    """Device buffers from the HIP runtime the library itself links."""

    def __init__(self):
        self.hip = C.CDLL("/opt/rocm/lib/libamdhip64.so.7")
        self.ptrs = []

    def put(self, arr):
        p = self.alloc(arr.nbytes)
        assert self.hip.hipMemcpy(C.c_void_p(p), arr.ctypes.data_as(C.c_void_p),
                                  C.c_size_t(arr.nbytes), 1) == 0  # host to device
        return p

    def alloc(self, nbytes):
        d = C.c_void_p()
        assert self.hip.hipMalloc(C.byref(d), C.c_size_t(max(nbytes, 8))) == 0
        self.ptrs.append(d.value)
        return d.value

    def get(self, p, out):
        assert self.hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(p),
                                  C.c_size_t(out.nbytes), 2) == 0  # device to host
        return out

    def free(self):
        for p in self.ptrs:
            self.hip.hipFree(C.c_void_p(p))
        self.ptrs = []


def _case(rng, nfeat):
    feats, hists, off = [], [], 0
    for _ in range(nfeat):
        nb = int(rng.choice([2, 3, 5, 17, 63, 64, 65, 130, 256]))
        mt = int(rng.integers(0, 3)) if nb > 2 else 0
        g = rng.normal(0, 1, nb) * (rng.random(nb) < 0.9)
        h = rng.random(nb) * 3 * (rng.random(nb) < 0.9)
        hist = np.empty(2 * nb)
        hist[0::2], hist[1::2] = g, h
        feats.append(BatchedFeature(off, nb, int(rng.integers(0, 2)), int(rng.integers(0, nb + 1)),
                                    0, int(nb > 2 and mt == 1), int(nb > 2 and mt == 2),
                                    int(nb > 2 and mt != 0), 0))
        hists.append(hist)
        off += 2 * nb
    return feats, np.concatenate(hists)


def _noalloc(be, dev, hist, feats, cfg, sg, sh, n):
    farr = np.frombuffer((BatchedFeature * len(feats))(*feats), dtype=np.uint8).copy()
    dh, df = dev.put(np.ascontiguousarray(hist)), dev.put(farr)
    do = dev.alloc(len(feats) * C.sizeof(SplitInfo))
    rc = be.lib.lgbm_hip_find_best_splits_noalloc(
        be.ctx, C.c_void_p(dh), C.c_int64(len(hist)), C.c_void_p(df), C.c_int32(len(feats)),
        C.byref(cfg), C.c_double(sg), C.c_double(sh), C.c_int32(n), C.c_void_p(do))
    out = (SplitInfo * len(feats))()
    raw = np.zeros(C.sizeof(out), np.uint8)
    dev.get(do, raw)
    C.memmove(out, raw.ctypes.data, raw.nbytes)
    return rc, list(out)


def _bits(si):
    return bytes(si)


def test_noalloc_matches_host_entry_twice():
    be = HipBackend(0)
    dev = Dev()
    try:
        rng = np.random.default_rng(2026)
        cfg = GainConfig.make(min_data_in_leaf=3, lambda_l1=0.3, lambda_l2=1.5,
                              min_gain_to_split=0.1)
        cfg.parent_output = 0.25
        for nfeat in (300, 41):  # the second call is smaller
            feats, hist = _case(rng, nfeat)
            sg, sh, n = float(rng.normal() * 5), float(rng.random() * 40 + 1), 4000
            want = be.find_best_splits_batched(hist, feats, cfg, sg, sh, n)
            rc, got = _noalloc(be, dev, hist, feats, cfg, sg, sh, n)
            assert rc == 0, be._err(be.ctx)
            assert len(got) == nfeat
            for j, (a, b) in enumerate(zip(got, want)):
                assert _bits(a) == _bits(b), (nfeat, j, a.as_dict(), b.as_dict())
    finally:
        dev.free()
        be.close()


def test_noalloc_limits_and_invalid_features():
    be = HipBackend(0)
    dev = Dev()
    try:
        rng = np.random.default_rng(7)
        cfg = GainConfig.make(min_data_in_leaf=3)
        feats, hist = _case(rng, 8)
        # above the maximum: refused before any work
        big = [feats[0]] * (MAX_FEATS + 1)
        rc, _ = _noalloc(be, dev, hist, big, cfg, 1.0, 10.0, 100)
        assert rc == -3, be._err(be.ctx)  # LGBM_HIP_ERR_CAPABILITY
        assert "exceeds" in be._err(be.ctx)
        # a region past the histogram: the host entry's LENGTH_MISMATCH, first feature named
        bad = list(feats)
        bad[5] = BatchedFeature(len(hist) - 2, 4, 0, 0, 0, 0, 0, 0, 0)
        rc, _ = _noalloc(be, dev, hist, bad, cfg, 1.0, 10.0, 100)
        assert rc == -1 and "feature 5" in be._err(be.ctx)
        bad[3] = BatchedFeature(0, 0, 0, 0, 0, 0, 0, 0, 0)
        rc, _ = _noalloc(be, dev, hist, bad, cfg, 1.0, 10.0, 100)
        assert rc == -4 and "feature 3" in be._err(be.ctx)  # RUNTIME: num_bin 0
        # the working memory is reset per call: a valid call right after succeeds
        want = be.find_best_splits_batched(hist, feats, cfg, 1.0, 10.0, 100)
        rc, got = _noalloc(be, dev, hist, feats, cfg, 1.0, 10.0, 100)
        assert rc == 0 and [_bits(a) for a in got] == [_bits(b) for b in want]
    finally:
        dev.free()
        be.close()
