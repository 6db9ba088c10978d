"""The oracle's logit soft cap (Gemma's cap * tanh(x / cap)) pinned against the reference's own
tests and against tanh itself.

* the reference's known-answer test (tests/test_kernels_gemma.py:8-48): x = randn(64) * 50 in
  f16, expected (tanh(x / 30) * 30) in f16, rtol = atol = 1e-2;
* its bounded invariant (tests/test_kernels_gemma.py:51-100): |out| <= cap on extreme inputs,
  f16's +-65504 included;
* every fp32 in [-20, 20] at cap 1 (the cap's tanh; constant +-1 outside): the absolute error
  against tanh in double, and the largest non-monotone drop, which the device sampler's single
  pass relies on (it thresholds raw logits and bounds the capped value below a threshold by
  the capped threshold plus cap * 2^-20);
* the sampler with a cap equals the sampler without one on logits capped beforehand."""
import numpy as np
import pytest

from oracle import sampler as O


def test_reference_known_answer():
    rng = np.random.default_rng(0)
    for _ in range(20):
        x = (rng.standard_normal(64) * 50.0).astype(np.float16)
        expected = (np.tanh(x.astype(np.float32) / 30.0) * 30.0).astype(np.float16)
        got = O.softcap_row(x.astype(np.float32), 30.0).astype(np.float16)
        np.testing.assert_allclose(got.astype(np.float32), expected.astype(np.float32),
                                   rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("cap", [30.0, 50.0, 1.0, 0.001])
def test_bounded_invariant(cap):
    rng = np.random.default_rng(1)
    inputs = [np.array([0.0, 1.0, -1.0, 100.0, -100.0, 29.999, -29.999, 1000.0], np.float32),
              (rng.standard_normal(256) * 500.0).astype(np.float32),
              np.full(64, 65504.0, np.float32), np.full(64, -65504.0, np.float32),
              np.array([np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45, -1e-45, 0.0, -0.0], np.float32)]
    for x in inputs:
        y = O.softcap_row(x, cap)
        assert np.all(np.abs(y) <= np.float32(cap)), (cap, x[np.abs(y) > cap][:4])
        assert np.all(np.isfinite(y))
    c = float(np.float32(cap))
    assert O.softcap_row(np.array([np.inf, -np.inf], np.float32), cap).tolist() == [c, -c]


def test_nan_stays_nan():
    y = O.softcap_row(np.array([np.nan, 1.0, np.nan], np.float32), 30.0)
    assert np.isnan(y[0]) and np.isnan(y[2]) and np.isfinite(y[1])


@pytest.mark.parametrize("cap", [30.0, 15.0, 1.5])
def test_close_to_tanh(cap):
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(200000) * cap * 3,
                        rng.standard_normal(20000) * 1e-3]).astype(np.float32)
    y = O.softcap_row(x, cap).astype(np.float64)
    ref = cap * np.tanh(x.astype(np.float64) / cap)
    assert np.max(np.abs(y - ref)) <= cap * 3e-7


def test_every_fp32_at_cap_one():
    """Exhaustive over [-20, 20]: error against tanh and the monotonicity drop bound."""
    r = O.check_softcap(-20.0, 20.0)
    assert r["count"] == O.key(20.0) - O.key(-20.0) + 1
    assert r["max_err"] <= 2.0 ** -22, r
    # the device's bound adds cap * 2^-20, which covers this drop and two roundings
    assert r["max_drop"] <= 2.0 ** -22, r
    # a plain monotone function would have no drop; this one does (so the bound is needed)
    assert r["max_drop"] > 0.0
    # outside [-20, 20] the value is exactly +-1, at or beyond everything inside
    y = O.softcap_row(np.array([-20.0, np.nextafter(np.float32(-20), np.float32(0)), 20.0,
                                np.nextafter(np.float32(20), np.float32(0))], np.float32), 1.0)
    assert y[0] == -1.0 and y[2] == 1.0 and y[1] >= -1.0 and y[3] <= 1.0


def test_sampler_caps_first():
    """sample(x, softcap=c) == sample(softcap_row(x, c)): the cap is the model's output."""
    rng = np.random.default_rng(3)
    B, V = 6, 3000
    x = (rng.standard_normal((B, V)) * 40).astype(np.float32)
    x[0, :50] = 1e4                      # saturated ties at +cap
    x[1, 7] = -np.inf
    prm = O.make_params(B, np.array([0.7, 0.0, 1.0, 0.5, 0.0, 1.2], np.float32),
                        np.array([50, 0, 5, 0, 1, 300], np.int32), 0.9, 0.05, 1.0, 0.0, 0.0)
    u = rng.uniform(1e-7, 1.0, (B, V)).astype(np.float32)
    capped = np.stack([O.softcap_row(r, 30.0) for r in x])
    a = O.sample(x, prm, u, num_logprobs=5, softcap=30.0)
    b = O.sample(capped, prm, u, num_logprobs=5)
    for key in ("token", "flags", "n_kept", "lp_ids", "lp_vals", "ranks"):
        assert np.array_equal(a[key], b[key]), key
    assert a["token"][0] < 50            # greedy over 50 tied maxima at +cap: lowest index


def test_round_f16_matches_numpy():
    """vwo_round_f16 against numpy's float32 -> float16 cast (round to nearest even) on random
    values of every magnitude, the f16 boundaries (max, overflow midpoint, subnormals, the
    smallest subnormal's half) and the specials."""
    rng = np.random.default_rng(4)
    bits = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 65536.0, -65520.0,
                        2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 3 * 2.0 ** -25,
                        2.0 ** -14, 2.0 ** -14 * (1 - 2 ** -11), 6.1e-5, 1e-8, 30.0, 29.99,
                        np.inf, -np.inf], np.float32)
    ties = (np.arange(1, 4000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)
    scaled = (rng.standard_normal(50000) * 30).astype(np.float32)
    for v in (x, special, ties, scaled):
        with np.errstate(over="ignore"):
            want = v.astype(np.float16).astype(np.float32)
        got = np.array([O.round_f16(float(t)) for t in v], np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            v[got.view(np.uint32) != want.view(np.uint32)][:5]
    assert np.isnan(O.round_f16(float("nan")))


def test_reference_known_answer_f16_store():
    """The reference's test compares f16 results; with the f16 store the cap's output is an f16
    value itself."""
    rng = np.random.default_rng(5)
    for _ in range(20):
        x = (rng.standard_normal(64) * 50.0).astype(np.float16).astype(np.float32)
        expected = (np.tanh(x / 30.0) * 30.0).astype(np.float16).astype(np.float32)
        got = O.softcap_row(x, 30.0, round_f16=True)
        assert np.array_equal(got, got.astype(np.float16).astype(np.float32))
        np.testing.assert_allclose(got, expected, rtol=1e-2, atol=1e-2)


def test_sampler_caps_first_f16_store():
    """sample(x, softcap=c, softcap_f16=True) == sample(f16(softcap_row(x, c))), including
    greedy rows whose maxima tie only after the f16 rounding (lowest index wins)."""
    rng = np.random.default_rng(6)
    B, V = 5, 4000
    x = (rng.standard_normal((B, V)) * 40).astype(np.float32)
    x[0, [100, 2000, 3000]] = [70.0, 70.01, 70.02]   # distinct in fp32, one f16 value once capped
    x[3, [5, 6]] = [60.0, 60.001]
    prm = O.make_params(B, np.array([0.0, 0.8, 1.0, 0.0, 0.6], np.float32),
                        np.array([0, 20, 0, 0, 100], np.int32), 0.9, 0.0, 1.0, 0.0, 0.0)
    u = rng.uniform(1e-7, 1.0, (B, V)).astype(np.float32)
    capped = np.stack([O.softcap_row(r, 30.0, round_f16=True) for r in x])
    assert capped[0, 100] == capped[0, 2000] == capped[0, 3000]
    assert O.softcap_row(x[0, [100, 2000]], 30.0)[0] != O.softcap_row(x[0, [100, 2000]], 30.0)[1]
    a = O.sample(x, prm, u, num_logprobs=3, softcap=30.0, softcap_f16=True)
    b = O.sample(capped, prm, u, num_logprobs=3)
    for key in ("token", "flags", "n_kept", "lp_ids", "lp_vals", "ranks"):
        assert np.array_equal(a[key], b[key]), key
    if capped[0].max() == capped[0, 100]:
        assert a["token"][0] == np.flatnonzero(capped[0] == capped[0].max())[0]
