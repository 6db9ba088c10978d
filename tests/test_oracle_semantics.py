"""Pins the oracle's sampling semantics on the CPU.

* the reference's own known-answer tests for this path (argmax / top-k / softmax kernels,
  ``tests/test_kernels_sample.py:13-145``, ``tests/test_kernels_attn.py:172-320``), replayed
  on the oracle;
* the greedy runner contract, ``vllm_webgpu/v1/model_runner.py:145`` (numpy argmax, lowest
  index on ties);
* every stage of the sampler against the independent float64 brute force in
  ``tests/bruteforce.py`` on random rows (bit-exact token ids off near ties);
* the distribution of the exponential race against ``p ~ softmax(x / T)``, the distribution
  the reference's CLI sampler draws from (``run_inference.py:383-390``), by a chi-square test.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import sampler as O
from tests import bruteforce as BF


# ---- the reference's known-answer tests ------------------------------------------------------

def test_kat_argmax_planted_77():
    # test_kernels_sample.py:13-16,43: 100.0 planted at 77 over V=128
    x = np.random.default_rng(0).normal(0, 1, (1, 128)).astype(np.float32)
    x[0, 77] = 100.0
    assert O.argmax(x)[0] == 77


def test_kat_argmax_unique_max_positions():
    # test_kernels_sample.py:122-145: unique max 50.0 at positions 0, 16, ..., 112
    for pos in range(0, 128, 16):
        x = np.zeros((1, 128), np.float32)
        x[0, pos] = 50.0
        assert O.argmax(x)[0] == pos


def test_kat_topk_five():
    # test_kernels_sample.py:55-58,93-101: values [10,9,8,7,6] at [77,3,100,50,22], descending
    x = np.random.default_rng(1).uniform(-1, 1, (1, 128)).astype(np.float32)
    ids = [77, 3, 100, 50, 22]
    for v, i in zip([10, 9, 8, 7, 6], ids):
        x[0, i] = v
    vals, got = O.topk(x, 5)
    assert got[0].tolist() == ids
    assert vals[0].tolist() == [10, 9, 8, 7, 6]


@pytest.mark.parametrize("family", ["normal", "constant", "spike", "wide"])
def test_kat_softmax_sums_to_one_and_shift_invariant(family):
    # test_kernels_attn.py:172-320: sums to 1, translation invariance for shifts {0, 5, -5, 100},
    # argmax preserved
    rng = np.random.default_rng(2)
    V = 1000
    x = {"normal": rng.normal(0, 1, V), "constant": np.full(V, 3.0),
         "spike": np.where(np.arange(V) == 17, 20.0, 0.0), "wide": rng.uniform(-30, 30, V)}[family]
    x = x.astype(np.float32)[None]
    p0, _, _ = O.softmax(x)
    assert abs(p0.astype(np.float64).sum() - 1.0) < 1e-5
    for s in (0.0, 5.0, -5.0, 100.0):
        ps, _, _ = O.softmax(x + np.float32(s))
        np.testing.assert_allclose(ps, p0, rtol=1e-5, atol=1e-7)
        assert np.argmax(ps) == np.argmax(x)


def test_softmax_closed_forms():
    V = 4096
    p, m, ls = O.softmax(np.full((1, V), 2.5, np.float32))
    np.testing.assert_allclose(p, 1.0 / V, rtol=1e-6)
    assert abs((m[0] + ls[0]) - (2.5 + np.log(V))) < 1e-5      # LSE = x + ln V
    # two-level row: a at n positions, b elsewhere
    x = np.zeros((1, V), np.float32)
    x[0, :10] = 3.0
    p, _, _ = O.softmax(x)
    e3 = np.exp(3.0)
    np.testing.assert_allclose(p[0, 0], e3 / (10 * e3 + V - 10), rtol=1e-6)
    # float64 brute force with temperature
    x = np.random.default_rng(3).normal(0, 3, (3, V)).astype(np.float32)
    for T in (1.0, 0.7):
        p, _, _ = O.softmax(x, T)
        y = (x / np.float32(T)).astype(np.float64)
        want = np.exp(y - y.max(1, keepdims=True))
        want /= want.sum(1, keepdims=True)
        np.testing.assert_allclose(p, want, rtol=1e-5, atol=1e-12)


def test_greedy_runner_contract_lowest_index():
    # model_runner.py:145: np.argmax -> first index of the max
    rng = np.random.default_rng(4)
    x = rng.integers(-3, 4, size=(64, 300)).astype(np.float32)   # many ties
    assert np.array_equal(O.argmax(x), np.argmax(x, axis=1))
    prm = O.make_params(64, temperature=0.0)
    assert np.array_equal(O.sample(x, prm)["token"], np.argmax(x, axis=1))


# ---- stages against the float64 brute force ----------------------------------------------------

def _random_rows(seed, n):
    rng = np.random.default_rng(seed)
    rows = []
    for _ in range(n):
        V = int(rng.choice([2, 3, 17, 64, 257, 1000, 4096]))
        x = rng.normal(0, rng.choice([0.5, 2.0, 4.0]), V).astype(np.float32)
        if rng.random() < 0.3:                       # fp16-representable values: many ties
            x = x.astype(np.float16).astype(np.float32)
        T = float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5]))
        k = int(rng.choice([0, 1, 5, 50, V]))
        p = float(rng.choice([1.0, 0.9, 0.5, 0.05, 0.0]))
        mp = float(rng.choice([0.0, 0.0, 0.05, 0.3]))
        pen = rng.random() < 0.5
        rep, pres, freq = (1.1, 0.5, 0.3) if pen else (1.0, 0.0, 0.0)
        H = int(rng.integers(0, 24))
        out = rng.integers(0, V + 1, H).astype(np.int32)            # V = padding
        prompt = rng.integers(0, V, int(rng.integers(0, 8))).astype(np.int32)
        u = (rng.integers(1, 2 ** 24, V) * 2.0 ** -24).astype(np.float32)
        rows.append((x, T, k, p, mp, rep, pres, freq, u, prompt, out))
    return rows


def _oracle_row(x, T, k, p, mp, rep, pres, freq, u, prompt, out):
    prm = O.make_params(1, T, k, p, mp, rep, pres, freq)
    pr = prompt[None] if prompt.size else None
    ou = out[None] if out.size else None
    return O.sample(x[None], prm, u[None], prompt_ids=pr, output_ids=ou)


def test_oracle_matches_float64_bruteforce():
    rows = _random_rows(5, 1500)
    skipped = 0
    for i, r in enumerate(rows):
        x, T, k, p, mp, rep, pres, freq, u, prompt, out = r
        want = BF.sample_row(x, T, k, p, mp, rep, pres, freq, u, prompt=prompt, output=out)
        got = _oracle_row(*r)
        near = (int(got["flags"][0]) & (O.FLAG_TOPP_NEAR_TIE | O.FLAG_RACE_NEAR_TIE)) != 0
        if near or not want["margin_ok"]:
            skipped += 1
            continue
        assert got["token"][0] == want["token"], (i, r[1:5], got["token"][0], want["token"])
        assert got["n_kept"][0] == want["n_kept"], (i, r[1:5], got["n_kept"][0], want["n_kept"])
    assert skipped < 0.03 * len(rows), skipped


def test_penalties_match_closed_form():
    rng = np.random.default_rng(6)
    V = 300
    x = rng.normal(0, 3, (4, V)).astype(np.float32)
    out = rng.integers(0, V, (4, 40)).astype(np.int32)
    out[:, :5] = out[:, 5:10]                     # duplicate tokens: counts > 1
    out[:, -3:] = V                              # padding
    prompt = rng.integers(0, V, (4, 12)).astype(np.int32)
    got = O.apply_penalties(x, prompt, out, 1.1, 0.5, 0.3)
    for b in range(4):
        want = BF.penalise(x[b], prompt[b], out[b], 1.1, 0.5, 0.3)
        assert np.array_equal(got[b], want)
    # identity penalties leave the row untouched
    assert np.array_equal(O.apply_penalties(x, prompt, out, 1.0, 0.0, 0.0), x)
    # empty history leaves the row untouched
    assert np.array_equal(O.apply_penalties(x, None, None, 1.3, 0.2, 0.1), x)


def test_greedy_rows_use_pre_temperature_penalised_argmax():
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (8, 500)).astype(np.float32)
    out = np.tile(np.argmax(x, 1)[:, None], (1, 3)).astype(np.int32)   # penalise the max
    prm = O.make_params(8, temperature=1e-6, top_k=3, top_p=0.5, repetition=1.5, presence=1.0)
    got = O.sample(x, prm, output_ids=out)
    pen = O.apply_penalties(x, None, out, 1.5, 1.0, 0.0)
    assert np.array_equal(got["token"], np.argmax(pen, 1))
    assert np.all(got["flags"] & O.FLAG_GREEDY)


def test_topk_keeps_all_ties_at_kth_and_k1_is_argmax():
    x = np.array([[1, 5, 3, 5, 5, 2, 5, 0]], np.float32)
    u = np.full((1, 8), 0.5, np.float32)
    r = O.sample(x, O.make_params(1, 1.0, top_k=2), u)
    assert r["n_kept"][0] == 4                   # four 5s tie at the 2nd largest
    r1 = O.sample(x, O.make_params(1, 1.0, top_k=1), u)
    assert r1["n_kept"][0] == 4 and r1["token"][0] == 1   # equal keys: lowest index
    rng = np.random.default_rng(8)
    y = rng.normal(0, 1, (16, 700)).astype(np.float32)
    uu = (rng.integers(1, 2 ** 24, (16, 700)) * 2.0 ** -24).astype(np.float32)
    r = O.sample(y, O.make_params(16, 0.8, top_k=1), uu)
    assert np.array_equal(r["token"], np.argmax(y, 1))


@pytest.mark.parametrize("V,p,kept", [(4, 0.5, 2), (8, 0.75, 6), (8, 0.25, 2), (5, 0.6, 4)])
def test_topp_removes_prefix_whose_mass_equals_one_minus_p(V, p, kept):
    # all-equal rows: the cumulative mass lands exactly on (1 - p) * total; vLLM masks
    # cumsum <= 1 - p, so the token that reaches the threshold exactly is removed
    x = np.zeros((1, V), np.float32)
    u = np.full((1, V), 0.5, np.float32)
    r = O.sample(x, O.make_params(1, 1.0, top_p=p), u)
    assert r["n_kept"][0] == kept
    assert r["token"][0] == V - kept                # equal keys: lowest surviving index


def test_topp_extremes_and_minp_one():
    rng = np.random.default_rng(9)
    x = rng.normal(0, 2, (8, 400)).astype(np.float32)
    u = (rng.integers(1, 2 ** 24, (8, 400)) * 2.0 ** -24).astype(np.float32)
    r = O.sample(x, O.make_params(8, 1.0, top_p=0.0), u)     # p -> 0: argmax survives alone
    assert np.array_equal(r["token"], np.argmax(x, 1)) and np.all(r["n_kept"] == 1)
    r = O.sample(x, O.make_params(8, 1.0, min_p=1.0), u)     # min_p = 1: only the max survives
    assert np.array_equal(r["token"], np.argmax(x, 1)) and np.all(r["n_kept"] == 1)
    r = O.sample(x, O.make_params(8, 1.0, top_p=1.0), u)     # p = 1: off
    assert np.all(r["n_kept"] == 400)


def test_constant_uniforms_pick_the_most_probable_survivor():
    # u == const  =>  q == const  =>  the race picks argmax p among survivors
    rng = np.random.default_rng(10)
    x = rng.normal(0, 2, (32, 900)).astype(np.float32)
    u = np.full((32, 900), 0.37, np.float32)
    r = O.sample(x, O.make_params(32, 0.9, top_k=40, top_p=0.8), u)
    assert np.array_equal(r["token"], np.argmax(x, 1))


# ---- distribution of the race ---------------------------------------------------------------

def _chi2_sf(stat, dof):
    from scipy.stats import chi2
    return float(chi2.sf(stat, dof))


@pytest.mark.parametrize("T,k,p", [(1.0, 0, 1.0), (0.6, 0, 1.0), (1.0, 3, 1.0), (1.0, 0, 0.7)])
def test_race_distribution_is_truncated_softmax(T, k, p):
    # run_inference.py:383-390 draws from softmax(x / T); the race must have that distribution
    # (restricted to the top-k / top-p survivors and renormalised)
    x = np.array([1.0, 0.2, -0.5, 2.0, 0.0, 1.5], np.float32)
    N = 40000
    rng = np.random.default_rng(11)
    u = (rng.integers(1, 2 ** 24, (N, x.size)) * 2.0 ** -24).astype(np.float32)
    r = O.sample(np.tile(x, (N, 1)), O.make_params(N, T, top_k=k, top_p=p), u)
    counts = np.bincount(r["token"], minlength=x.size).astype(np.float64)
    y = (x / np.float32(T)).astype(np.float64)
    w = np.exp(y - y.max())
    keep = np.ones(x.size, bool)
    if k:
        keep &= y >= np.sort(y)[::-1][k - 1]
    if p < 1:
        order = np.argsort(y, kind="stable")
        order = order[keep[order]]
        c = np.cumsum(w[order]) / w[keep].sum()
        rem = c <= np.float32(1) - np.float32(p)
        rem[-1] = False
        keep[order[rem]] = False
    w = np.where(keep, w, 0.0)
    expect = N * w / w.sum()
    assert np.all(counts[~keep] == 0)
    stat = (((counts - expect) ** 2)[keep] / expect[keep]).sum()
    assert _chi2_sf(stat, int(keep.sum()) - 1) > 1e-4, (counts, expect)


# ---- logprobs ------------------------------------------------------------------------------

def test_raw_logprobs_match_float64_log_softmax():
    rng = np.random.default_rng(12)
    B, V, L = 6, 3000, 20
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    x[0, 10:20] = x[0].max()                                # ties in the top-L
    u = (rng.integers(1, 2 ** 24, (B, V)) * 2.0 ** -24).astype(np.float32)
    r = O.sample(x, O.make_params(B, 1.0, top_p=0.9), u, num_logprobs=L)
    for b in range(B):
        ls = BF.log_softmax(x[b])
        s = r["token"][b]
        assert r["lp_ids"][b, 0] == s
        np.testing.assert_allclose(r["lp_vals"][b, 0], ls[s], rtol=1e-5, atol=1e-6)
        top = BF.topk_desc(x[b], L)
        assert np.array_equal(r["lp_ids"][b, 1:], top)
        np.testing.assert_allclose(r["lp_vals"][b, 1:], ls[top], rtol=1e-5, atol=1e-6)
        assert r["ranks"][b] == int((x[b] >= x[b, s]).sum())
