"""The greedy kernel's two-candidate window against the reference's full grid
scan (converter/greedy.py:80-95), on the CPU in float32.

For one column of one row the reference evaluates, for every grid value g
in increasing order, ne = e + (g - q) s and cost = ne*ne*h + 2*ne*cross and
keeps the first minimum (codes start at q, best cost at 1e30).  The kernel
(ldlq.hip, greedy_decide) evaluates only g0 = clamp(floor(t), qmin, qmax-1)
and g0 + 1 around the continuous minimiser t = q - (cross/h + e)/s, and
takes that answer only inside a guard: |cross| <= 128 h s, |t| < 2^16,
h in [2^-60, 2^30], s^2 in [2^-40, 2^30].  Inside the guard the cost's
fp32 rounding is far below the gap h s^2 between neighbouring grid
values, so no other grid value can tie or beat the better of the two.
These tests check that claim on random and adversarial inputs (near-ties at
half-integers, the guard's edges, clamped windows), and that a loosened
guard does produce mismatches, so the check has teeth.
"""
import numpy as np
import pytest

f32 = np.float32


def full_scan(e, q, s, h, c, qmin, qmax):
    best = np.full(e.shape, f32(1e30), dtype=f32)
    bq = q.copy()
    for g in range(qmin, qmax + 1):
        g = f32(g)
        ne = e + (g - q) * s
        cost = ne * ne * h + f32(2) * ne * c
        better = cost < best
        best = np.where(better, cost, best)
        bq = np.where(better, g, bq)
    return np.clip(bq, qmin, qmax)


def window(e, q, s, h, c, qmin, qmax, gamma=128.0, tmax=65536.0):
    ih = (f32(1) / h).astype(f32)
    inv_s = (f32(1) / s).astype(f32)
    # fmaf(c, ih, e) rounded once
    t = q - (c.astype(np.float64) * ih + e).astype(f32) * inv_s
    g0 = np.clip(np.floor(t), qmin, qmax - 1).astype(f32)
    g1 = g0 + f32(1)
    n0 = e + (g0 - q) * s
    n1 = e + (g1 - q) * s
    c0 = n0 * n0 * h + f32(2) * n0 * c
    c1 = n1 * n1 * h + f32(2) * n1 * c
    bq = np.where(c1 < c0, g1, g0)
    hg = np.where((h >= 2.0 ** -60) & (h <= 2.0 ** 30), h, np.nan).astype(f32)
    s2 = s.astype(np.float64) ** 2
    sg = np.where((s > 0) & (s2 >= 2.0 ** -40) & (s2 <= 2.0 ** 30), f32(gamma) * s, np.nan).astype(f32)
    with np.errstate(invalid="ignore"):
        ok = (np.abs(c) <= hg * sg) & (np.abs(t) < f32(tmax))
    return bq, ok


def cases(rng, n, qmin, qmax, mode):
    h = (2.0 ** rng.uniform(-60, 30, n)).astype(f32)
    s = (2.0 ** rng.uniform(-20, 15, n)).astype(f32)
    q = rng.integers(qmin, qmax + 1, n).astype(f32)
    if mode == "typical":
        e = (s * rng.uniform(-1, 1, n)).astype(f32)
        c = (h * s * rng.uniform(-20, 20, n)).astype(f32)
    elif mode == "ties":          # t within 1e-5 of a half-integer
        e = (s * rng.uniform(-3, 3, n)).astype(f32)
        tt = rng.integers(qmin - 3, qmax + 3, n) + 0.5 + rng.uniform(-1e-5, 1e-5, n)
        c = (-(h.astype(np.float64)) * ((tt - q) * s + e)).astype(f32)
    elif mode == "guard_edge":    # |cross| around 128 h s, large errors
        e = (s * rng.uniform(-1, 1, n) * 10.0 ** rng.uniform(0, 4.8, n)).astype(f32)
        c = (h * s * rng.uniform(-130, 130, n)).astype(f32)
    else:                         # clamped windows
        e = (s * rng.uniform(-70000, 70000, n)).astype(f32)
        c = (h * s * rng.uniform(-128, 128, n)).astype(f32)
    return e, q, s, h, c


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("mode", ["typical", "ties", "guard_edge", "clamped"])
def test_window_equals_full_scan_inside_guard(bits, mode):
    qmin, qmax = (-8, 7) if bits == 4 else (-128, 127)
    rng = np.random.default_rng(bits * 100 + len(mode))
    n = 200_000 if bits == 4 else 50_000
    e, q, s, h, c = cases(rng, n, qmin, qmax, mode)
    with np.errstate(all="ignore"):
        want = full_scan(e, q, s, h, c, qmin, qmax)
        got, ok = window(e, q, s, h, c, qmin, qmax)
    assert ok.mean() > 0.5                    # the guard leaves most inputs to the window
    assert not np.any((got != want) & ok)


def test_loose_guard_is_caught():
    qmin, qmax = -8, 7
    rng = np.random.default_rng(7)
    n = 200_000
    h = (2.0 ** rng.uniform(-60, 30, n)).astype(f32)
    s = (2.0 ** rng.uniform(-20, 15, n)).astype(f32)
    q = rng.integers(qmin, qmax + 1, n).astype(f32)
    e = (s * rng.uniform(-1, 1, n) * 10.0 ** rng.uniform(0, 9, n)).astype(f32)
    tt = rng.integers(qmin - 3, qmax + 3, n) + 0.5 + rng.uniform(-1e-3, 1e-3, n)
    c = (-(h.astype(np.float64)) * ((tt - q) * s + e)).astype(f32)
    with np.errstate(all="ignore"):
        want = full_scan(e, q, s, h, c, qmin, qmax)
        got, ok = window(e, q, s, h, c, qmin, qmax, gamma=2.0 ** 30, tmax=2.0 ** 40)
    assert np.any((got != want) & ok)


def test_dead_channel_takes_first_grid_value():
    # h = 0 and cross = 0: every cost is 0, the scan keeps the first grid
    # value; the window's t is NaN, outside the guard, so the kernel scans
    e = np.zeros(4, dtype=f32)
    q = np.array([3, -2, 0, 7], dtype=f32)
    s = np.full(4, 0.1, dtype=f32)
    h = np.zeros(4, dtype=f32)
    c = np.zeros(4, dtype=f32)
    with np.errstate(all="ignore"):
        assert np.all(full_scan(e, q, s, h, c, -8, 7) == -8)
        _, ok = window(e, q, s, h, c, -8, 7)
    assert not ok.any()
