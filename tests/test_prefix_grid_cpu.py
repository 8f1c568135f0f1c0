"""The threshold scans' grid prefix (prefix_grid in lightgbm_rs_amd/csrc/scan.h), modelled
lane by lane on the CPU: for cells that are exact multiples of one unit except one
arbitrary cell, and any carry, every lane's sum must equal the reference's sequential
f64 sum bit for bit (learner scans accumulate candidates in order from kEpsilon,
kernels/split.rs:9078-9277).  The model follows the kernel step for step: an exact
prefix of the unit cells, each lane's step from the last rounding step, a TwoSum test,
and the first rounding (or odd) lane becomes the next base.  A planted mistake (the
prefix taken as exact without the rounding steps) must fail.
"""
import struct

import numpy as np

K_EPS = 1e-15
W = 64


def bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def two_sum_exact(a, b, s):
    bv = s - a
    av = s - bv
    return ((a - av) + (b - bv)) == 0.0


def model(vals, cnt, odd, carry, replay=True):
    v = [vals[i] if i < cnt else 0.0 for i in range(W)]
    unit = [v[i] if (i < cnt and i != odd) else 0.0 for i in range(W)]
    p, acc = [], 0.0
    for i in range(W):
        acc = acc + unit[i]  # exact: unit multiples well below 2^53 units
        p.append(acc)
    q = [0.0] + p[:-1]
    out = [None] * W
    ts, tp, t = carry, 0.0, -1
    while True:
        a = [ts if q[i] == tp else ts + (q[i] - tp) for i in range(W)]
        n = [a[i] + v[i] for i in range(W)]
        bad = [replay and (t < i < cnt) and (i == odd or not two_sum_exact(a[i], v[i], n[i]))
               for i in range(W)]
        j = next((i for i in range(W) if bad[i]), W)
        for i in range(W):
            if t < i < cnt and i <= j:
                out[i] = n[i]
        if j == W:
            return out[:cnt]
        ts, tp, t = n[j], p[j], j


def sequential(vals, cnt, carry):
    out, s = [], carry
    for i in range(cnt):
        s = s + vals[i]
        out.append(s)
    return out


def cases(n, seed):
    rng = np.random.default_rng(seed)
    for case in range(n):
        scale = float(np.float32(rng.uniform(1e-4, 10.0)))
        u = float(np.spacing(np.float32(scale)))
        cnt = int(rng.integers(1, W + 1))
        kind = case % 3
        if kind == 0:  # hessians: nonnegative from kEpsilon
            ks = rng.integers(0, 1 << int(rng.integers(1, 26)), size=cnt)
            ks[rng.random(cnt) < 0.3] = 0
            carry = K_EPS if rng.random() < 0.5 else K_EPS + float(rng.integers(0, 1 << 20)) * u
        elif kind == 1:  # gradients: signed from 0 or an on-grid carry
            ks = rng.integers(-(1 << 20), 1 << 20, size=cnt)
            carry = 0.0 if rng.random() < 0.5 else float(rng.integers(-(1 << 30), 1 << 30)) * u
        else:  # an arbitrary carry (after the fixed cell)
            ks = rng.integers(-(1 << 22), 1 << 22, size=cnt)
            carry = float(rng.normal()) * float(10.0 ** rng.integers(-6, 6))
        vals = [float(k) * u for k in ks]
        odd = -1
        if rng.random() < 0.4:
            odd = int(rng.integers(0, cnt))
            vals[odd] = float(rng.normal()) * float(10.0 ** rng.integers(-3, 4))
            if rng.random() < 0.1:
                vals[odd] = -0.0
        yield vals, cnt, odd, carry


def test_grid_prefix_equals_sequential_sums():
    for vals, cnt, odd, carry in cases(3000, 1):
        out = model(vals, cnt, odd, carry)
        ref = sequential(vals, cnt, carry)
        assert [bits(a) for a in out] == [bits(b) for b in ref], (cnt, odd, carry)


def test_planted_mistake_without_rounding_steps_fails():
    """The exact prefix alone (no replay of the rounding steps) misses the kEpsilon
    start's roundings and the odd cell: the check must catch it."""
    mismatches = 0
    for vals, cnt, odd, carry in cases(300, 2):
        out = model(vals, cnt, odd, carry, replay=False)
        ref = sequential(vals, cnt, carry)
        mismatches += [bits(a) for a in out] != [bits(b) for b in ref]
    assert mismatches > 50
