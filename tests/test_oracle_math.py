"""Pins the oracle's sampler arithmetic (CPU only): exp_det / log_det against libm in float64,
the integer masses and the 128-bit threshold against Python's exact rationals, and the order
keys against the float order."""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import sampler as O


@pytest.mark.parametrize("lo,hi,stride", [(-80.0, 80.0, 1009), (-1e-3, 1e-3, 7), (-80.0, -70.0, 13)])
def test_exp_det_within_one_ulp(lo, hi, stride):
    r = O.check_exp(lo, hi, stride)
    assert r["count"] > 100_000
    assert r["max_ulp"] <= 1, r


@pytest.mark.parametrize("lo,hi,stride", [(1.0e-38, 1.0, 1009), (0.5, 2.0, 7), (5.9604645e-08, 1e-6, 3)])
def test_log_det_within_one_ulp(lo, hi, stride):
    r = O.check_log(lo, hi, stride)
    assert r["count"] > 100_000
    assert r["max_ulp"] <= 1, r


def test_exp_log_special_values():
    assert O.exp_det(0.0) == 1.0
    assert O.exp_det(-0.0) == 1.0
    assert O.exp_det(-80.5) == 0.0
    assert O.exp_det(float("nan")) == 0.0
    assert O.log_det(1.0) == 0.0
    # exact powers of two: log(2^e) = e*ln2 rounded once
    for e in (-24, -10, -1, 1, 5):
        want = np.float32(e * np.log(2.0))
        assert abs(O.log_det(2.0 ** e) - want) <= abs(np.spacing(want))
    # exp of exact multiples of ln2 hits the power of two within one ulp
    for n in (-20, -3, 3, 20):
        v = O.exp_det(np.float32(n * np.log(2.0)))
        assert abs(v / 2.0 ** n - 1.0) < 2.5e-7


def test_mass_is_floor_of_e_times_2_pow_44():
    rng = np.random.default_rng(1)
    es = np.concatenate([rng.random(2000, dtype=np.float32),
                         np.array([0.0, 1.0, 2.0 ** -44, 2.0 ** -45, 0.5, np.float32(1) - np.float32(2 ** -24)],
                                  np.float32)])
    for e in es:
        want = int(Fraction(float(e)) * 2 ** 44)
        assert O.mass(float(e)) == want, e


def test_scale_floor_is_exact_floor_q_times_w():
    rng = np.random.default_rng(2)
    for _ in range(3000):
        q = np.float32(rng.random())
        W = int(rng.integers(1, 2 ** 63 - 1, dtype=np.int64))
        want = int(Fraction(float(q)) * W)  # int() of a positive Fraction is floor
        assert O.scale_floor(float(q), W) == want, (q, W)
    assert O.scale_floor(0.0, 12345) == 0
    assert O.scale_floor(1.0, 2 ** 63) == 2 ** 63


def test_order_key_is_monotone_and_folds_signed_zero():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 1e3, 4000).astype(np.float32),
                        np.array([np.inf, -np.inf, 0.0, -0.0, 1e-45, -1e-45, 3.4e38, -3.4e38],
                                 np.float32)])
    keys = np.array([O.key(float(v)) for v in x], np.uint64)
    order = np.argsort(x, kind="stable")
    ks = keys[order]
    assert np.all(ks[1:] >= ks[:-1])
    # equal keys exactly for equal values (with -0 == +0)
    xs = x[order]
    same = xs[1:] == xs[:-1]
    assert np.array_equal(ks[1:][same], ks[:-1][same])
    assert O.key(0.0) == O.key(-0.0)
    assert O.key(float("nan")) == 0
    assert O.key(-np.inf) > 0
