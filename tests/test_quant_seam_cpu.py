"""The drop-in quantizer seam on the CPU (no device): the arithmetic behind
lgbm_hip_set_dequantized_gradients.

The reference quantizes in place (quantize_grad_hess_in_place, gbdt.rs:43-62,
945-960): every g / h becomes f32(q * scale).  An adapter that uploads those arrays
must recover q, not quantize them again.  Pinned here at configs[1]'s size (10.5M
rows) with a full-mantissa max |h|:
  * round(v / scale) recovers the oracle's q on every row and f32(q * scale) == v
    (the device kernel k_requant computes exactly this);
  * quantizing the dequantized values again with the same seed is NOT the identity
    (it moves some q), which is why the seam recovers instead of re-quantizing."""
import numpy as np

from oracle import oracle

N = 10_500_000
SEED = ((7 << 20) ^ 0x51702010)  # iteration 7's seed (gbdt.rs:950)


# max |h|: a full 24-bit mantissa whose f32(3 * max/4) rounds up by 1.26e-7 of the
# scale, so a dequantized q_h = 3 reads back as 3 + 1.26e-7
MAX_H = np.float32(0.23707023)
# rows whose hessian draw of SEED's xorshift stream (gradient_discretizer.rs:173-188:
# grad draw, then hess draw) lies within 1.4e-8 of 1
NEAR_ONE_ROWS = (4045883, 1024877)


def _inputs():
    rng = np.random.default_rng(20261202)
    g = rng.standard_normal(N, dtype=np.float32)
    h = (rng.random(N, dtype=np.float32) * MAX_H).astype(np.float32)
    h[12345] = MAX_H
    for r in NEAR_ONE_ROWS:  # q_h = 3 (2.9 + a draw near 1 truncates to 3)
        h[r] = np.float32(2.9 * float(MAX_H) / 4)
    return g, h


def test_recovery_is_exact_at_config1_size():
    g, h = _inputs()
    dg, dh, disc, (gs, hs) = oracle.quantize(g, h, bins=4, stochastic=True, seed=SEED)
    qg, qh = disc[1::2].astype(np.int64), disc[0::2].astype(np.int64)
    rg = np.rint(dg.astype(np.float64) / gs).astype(np.int64)
    rh = np.rint(dh.astype(np.float64) / hs).astype(np.int64)
    assert np.array_equal(rg, qg)
    assert np.array_equal(rh, qh)
    assert np.array_equal((rg * gs).astype(np.float32).view(np.uint32), dg.view(np.uint32))
    assert np.array_equal((rh * hs).astype(np.float32).view(np.uint32), dh.view(np.uint32))
    assert qg.min() >= -2 and qg.max() <= 2 and qh.min() >= 0 and qh.max() <= 4


def test_requantizing_dequantized_values_moves_q():
    u = oracle.xorshift_u01(SEED ^ 0x9E3779B97F4A7C15, 2 * N)
    for r in NEAR_ONE_ROWS:
        assert 1.0 - u[2 * r + 1] < 1.5e-8
    g, h = _inputs()
    dg, dh, disc, _ = oracle.quantize(g, h, bins=4, stochastic=True, seed=SEED)
    _, _, disc2, _ = oracle.quantize(dg, dh, bins=4, stochastic=True, seed=SEED)
    moved = np.nonzero(disc2 != disc)[0]
    assert set(2 * r for r in NEAR_ONE_ROWS) <= set(moved.tolist())
    for r in NEAR_ONE_ROWS:
        assert disc[2 * r] == 3 and disc2[2 * r] == 4
