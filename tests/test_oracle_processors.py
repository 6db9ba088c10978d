"""The oracle's logits processors (vLLM-v1: allowed-token mask, bans from bad words and
min-tokens, logit bias; all ahead of the penalties) against an independent numpy restatement,
known answers that fix the order of operations, and the raw-logprob contract (processors do not
touch raw logprobs)."""
import numpy as np
import pytest

from oracle import sampler as O
from tests import bruteforce as BF


def _bits(allowed):
    """bool [B, V] -> uint32 [B, ceil(V/32)] bitmask, bit set = allowed."""
    B, V = allowed.shape
    W = (V + 31) // 32
    out = np.zeros((B, W), np.uint32)
    for b in range(B):
        for i in np.nonzero(allowed[b])[0]:
            out[b, i >> 5] |= np.uint32(1 << (i & 31))
    return out


def _random_adjust(rng, B, V, width):
    ids = rng.integers(-2, V + 2, size=(B, width)).astype(np.int32)      # some padding ids
    vals = rng.normal(0, 2, size=(B, width)).astype(np.float32)
    vals[rng.random((B, width)) < 0.3] = -np.inf                          # bans
    for b in range(B):                                                    # one finite entry per token
        seen = set()
        for j in range(width):
            t = int(ids[b, j])
            if vals[b, j] != -np.inf:
                if t in seen:
                    vals[b, j] = -np.inf
                seen.add(t)
    return ids, vals


def test_adjustments_match_numpy():
    rng = np.random.default_rng(7)
    B, V = 16, 300
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    ids, vals = _random_adjust(rng, B, V, 24)
    allowed = rng.random((B, V)) < 0.8
    got = O.apply_adjustments(x, _bits(allowed), ids, vals)
    for b in range(B):
        exp = BF.process(x[b], allowed[b], ids[b], vals[b])
        np.testing.assert_array_equal(got[b].view(np.uint32), exp.view(np.uint32))


def test_sampling_with_processors_matches_bruteforce():
    rng = np.random.default_rng(11)
    B, V = 400, 64
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    ids, vals = _random_adjust(rng, B, V, 6)
    allowed = rng.random((B, V)) < 0.7
    allowed[:, 0] = True
    T = rng.uniform(0.3, 1.5, B).astype(np.float32)
    T[::5] = 0.0
    k = rng.choice([0, 5, 20], B).astype(np.int32)
    p = rng.choice([1.0, 0.9, 0.6], B).astype(np.float32)
    mp = rng.choice([0.0, 0.05], B).astype(np.float32)
    rep = rng.choice([1.0, 1.3], B).astype(np.float32)
    hist = rng.integers(0, V, (B, 8)).astype(np.int32)
    u = (rng.integers(1, 2 ** 24, (B, V)) * 2.0 ** -24).astype(np.float32)
    prm = O.make_params(B, T, k, p, mp, rep, 0.2, 0.1)
    res = O.sample(x, prm, u, output_ids=hist, allowed=_bits(allowed), adjust_ids=ids,
                   adjust_vals=vals)
    checked = 0
    for b in range(B):
        bf = BF.sample_row(x[b], T[b], k[b], p[b], mp[b], rep[b], 0.2, 0.1, u[b], output=hist[b],
                           allowed=allowed[b], adj_ids=ids[b], adj_vals=vals[b])
        if not bf["margin_ok"]:
            continue
        checked += 1
        assert res["token"][b] == bf["token"], b
        assert allowed[b][res["token"][b]], b
    assert checked > 350


def _one(x, T=0.0, hist=None, rep=1.0, allowed=None, ids=None, vals=None, u=None):
    x = np.asarray([x], np.float32)
    V = x.shape[1]
    prm = O.make_params(1, T, 0, 1.0, 0.0, rep, 0.0, 0.0)
    al = None if allowed is None else _bits(np.asarray([allowed], bool))
    ai = None if ids is None else np.asarray([ids], np.int32)
    av = None if vals is None else np.asarray([vals], np.float32)
    h = None if hist is None else np.asarray([hist], np.int32)
    uu = None if u is None else np.asarray([u], np.float32)
    return int(O.sample(x, prm, uu, output_ids=h, allowed=al, adjust_ids=ai, adjust_vals=av)["token"][0])


def test_known_answers():
    x = [1.0, 5.0, 3.0, 4.0]
    assert _one(x) == 1
    assert _one(x, ids=[1], vals=[-np.inf]) == 3                          # banned argmax
    assert _one(x, ids=[0], vals=[10.0]) == 0                             # bias lifts a token
    assert _one(x, ids=[1, 1], vals=[10.0, -np.inf]) == 3                 # a ban beats a bias
    assert _one(x, allowed=[True, False, True, False]) == 2               # allowed-token mask
    assert _one(x, T=1.0, allowed=[False, False, True, False],
                u=[0.5, 0.5, 0.5, 0.5]) == 2                              # only one token left
    assert _one(x, ids=[7, -1], vals=[100.0, 100.0]) == 1                 # padding ids ignored


def test_bias_applies_before_the_penalties():
    # token 0 is in the output history and biased by +1, repetition 2:
    # bias first: (3 + 1) / 2 = 2 < 2.4 -> token 1; penalty first would give 3 / 2 + 1 = 2.5
    assert _one([3.0, 2.4], hist=[0], rep=2.0, ids=[0], vals=[1.0]) == 1
    assert _one([3.0, 2.4], hist=[0], rep=2.0) == 1
    assert _one([3.0, 2.4], ids=[0], vals=[1.0]) == 0


def test_processors_leave_raw_logprobs_alone():
    rng = np.random.default_rng(3)
    B, V, L = 8, 200, 5
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    ids = np.tile(np.argsort(-x, axis=1)[:, :3].astype(np.int32), 1)    # ban each row's top 3
    vals = np.full(ids.shape, -np.inf, np.float32)
    prm = O.make_params(B, 0.0, 0, 1.0, 0.0, 1.0, 0.0, 0.0)
    a = O.sample(x, prm, None, num_logprobs=L)
    b = O.sample(x, prm, None, num_logprobs=L, adjust_ids=ids, adjust_vals=vals)
    np.testing.assert_array_equal(a["lp_ids"][:, 1:], b["lp_ids"][:, 1:])
    np.testing.assert_array_equal(a["lp_vals"][:, 1:], b["lp_vals"][:, 1:])
    assert (b["token"] == np.argsort(-x, axis=1)[:, 3]).all()          # best unbanned token
