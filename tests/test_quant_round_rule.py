"""CPU: the rounding rule the GPU quantisers use (csrc/device_common.hpp
quant_round), restated in numpy float32, equals rint of the correctly
rounded quotient rint(fl(x / s)) -- what torch computes -- for reciprocals
anywhere within 1 ulp of 1/s (v_rcp_f32's bound), on quotients built to sit
within a few ulps of half-integers and on random ones, for |x / s| up to
256. A planted variant without the near-tie fallback must fail."""
from __future__ import annotations

import numpy as np

F = np.float32


def _rule(x, s, r, fallback=True):
    y = (x * r).astype(F)
    k = np.rint(y)
    near = np.abs((y - k).astype(F)) >= F(0.5) - F(2.0 ** -12)
    if not fallback:
        return k
    return np.where(near, np.rint((x / s).astype(F)), k)


def _cases(rng, n=200_000, qmax=127):
    s = (rng.uniform(1e-3, 10.0, n)).astype(F)
    k = rng.integers(-qmax, qmax, n).astype(F)
    ulps = rng.integers(-4, 5, n)
    x = ((k + F(0.5)) * s).astype(F)
    x = np.nextafter(x, np.where(ulps > 0, np.inf, -np.inf).astype(F)).astype(F)   # within ulps of a tie
    xr = (rng.uniform(-qmax, qmax, n) * s).astype(F)
    return np.concatenate([x, xr]), np.concatenate([s, s])


def test_rule_equals_correctly_rounded_quotient():
    rng = np.random.default_rng(7)
    for qmax in (7, 127, 255):
        x, s = _cases(rng, qmax=qmax)
        want = np.rint((x / s).astype(F))
        r0 = (F(1.0) / s).astype(F)
        for shift in (-1, 0, 1):   # every reciprocal within 1 ulp of the correctly rounded one
            r = r0 if shift == 0 else np.nextafter(r0, F(np.inf) if shift > 0 else F(-np.inf)).astype(F)
            assert np.array_equal(_rule(x, s, r), want), (qmax, shift)


def test_planted_no_fallback_fails():
    rng = np.random.default_rng(8)
    x, s = _cases(rng, qmax=127)
    r = np.nextafter((F(1.0) / s).astype(F), F(np.inf)).astype(F)
    assert not np.array_equal(_rule(x, s, r, fallback=False), np.rint((x / s).astype(F)))


def test_near_tie_window_forms_agree():
    """|y - k| >= 0.5 - 2^-12 (the kernels' form) selects the same y as
    ||y - k| - 0.5| <= 2^-12 for k = rint(y), |y - k| <= 0.5: on fp32 values
    around half-integers (every ulp step within 2^-11 of them, |y| up to
    300), random ones, exact ties and integers."""
    rng = np.random.default_rng(3)
    centers = np.arange(-300, 300, dtype=F) + F(0.5)
    ys = [centers, np.arange(-300, 300, dtype=F)]
    for c in (centers[::7], centers[3::11]):
        y = c.copy()
        for _ in range(600):                      # walk ulp by ulp out of the window
            y = np.nextafter(y, F(np.inf)).astype(F)
            ys.append(y.copy())
        y = c.copy()
        for _ in range(600):
            y = np.nextafter(y, F(-np.inf)).astype(F)
            ys.append(y.copy())
    ys.append(rng.uniform(-300, 300, 200_000).astype(F))
    y = np.concatenate(ys).astype(F)
    k = np.rint(y)
    d = np.abs((y - k).astype(F))
    assert (d <= F(0.5)).all()
    old = np.abs((d - F(0.5)).astype(F)) <= F(2.0 ** -12)
    new = d >= F(0.5) - F(2.0 ** -12)
    assert np.array_equal(old, new)
    assert new.any() and (~new).any()

