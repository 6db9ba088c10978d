"""Brute-force float64 restatement of the sampler, written independently of ``oracle/``.

It follows the vLLM-v1 Sampler flow that the reference plugin hands sampling to
(``docs/superpowers/specs/2026-06-29-vllm-webgpu-design.md:451``) in the plainest form:
probabilities in float64 (``numpy.exp``/``numpy.log``), a stable sort and a float64 cumulative
sum for top-p, ``p / q`` with ``q = -ln u`` for the exponential race.  It shares none of the
oracle's integer-mass, order-key or polynomial machinery, so a dropped term, a flipped
comparison or a transposed operand in either one shows up as a token mismatch.

Float64 cannot decide rows that sit on a boundary, so every result carries a ``margin_ok``
flag: False when the top-p cut, the min-p cut or the race's two best candidates are closer than
a relative 1e-6 -- the tests skip those rows and bound how many there are.
"""
from __future__ import annotations

import numpy as np

EPS_GREEDY = np.float32(1e-5)
MARGIN = 1e-6


def penalise(x, prompt, output, rep, pres, freq):
    """Penalties on fp32 logits, in the vLLM-v1 order: repetition on prompt|output tokens
    (positive logits times fl(1/r), others times r), then ``- freq * count`` then
    ``- pres * (count > 0)`` on output counts.  History ids outside [0, V) are padding."""
    x = np.asarray(x, np.float32).copy()
    V = x.size
    rep, pres, freq = np.float32(rep), np.float32(pres), np.float32(freq)
    if rep == 1 and pres == 0 and freq == 0:
        return x
    cnt = np.zeros(V, np.int64)
    seen = np.zeros(V, bool)
    for t in (output if output is not None else ()):
        if 0 <= t < V:
            cnt[t] += 1
    for t in (prompt if prompt is not None else ()):
        if 0 <= t < V:
            seen[t] = True
    seen |= cnt > 0
    inv = np.float32(1.0) / rep
    x = np.where(seen, np.where(x > 0, x * inv, x * rep), x).astype(np.float32)
    x = (x - freq * cnt.astype(np.float32)).astype(np.float32)
    x = (x - pres * (cnt > 0).astype(np.float32)).astype(np.float32)
    return x


def first_argmax(x):
    """Lowest index of the largest non-NaN value (numpy argmax semantics, NaN never wins)."""
    x = np.asarray(x)
    ok = ~np.isnan(x)
    if not ok.any():
        return 0
    m = x[ok].max()
    return int(np.nonzero(ok & (x == m))[0][0])


def process(x, allowed=None, adj_ids=None, adj_vals=None):
    """vLLM-v1 logits processors ahead of the penalties: disallowed tokens (``allowed`` is a
    bool [V] here) and tokens listed with -inf become -inf, a token listed with a finite value
    gets it added in fp32.  Ids outside [0, V) are padding."""
    x = np.asarray(x, np.float32).copy()
    V = x.size
    if allowed is not None:
        x[~np.asarray(allowed, bool)] = -np.inf
    if adj_ids is not None:
        ids = np.asarray(adj_ids)
        vals = np.asarray(adj_vals, np.float32)
        ok = (ids >= 0) & (ids < V)
        banned = set(int(t) for t, v in zip(ids[ok], vals[ok]) if v == -np.inf)
        for t, v in zip(ids[ok], vals[ok]):
            if int(t) not in banned:
                x[t] = np.float32(x[t] + v)
        for t in banned:
            x[t] = -np.inf
    return x


def sample_row(x0, T, k, p, min_p, rep, pres, freq, u, prompt=None, output=None, allowed=None,
               adj_ids=None, adj_vals=None):
    """Returns dict(token, n_kept, margin_ok) for one row."""
    x = penalise(process(x0, allowed, adj_ids, adj_vals), prompt, output, rep, pres, freq)
    V = x.size
    T = np.float32(T)
    if not (T >= EPS_GREEDY):
        return dict(token=first_argmax(x), n_kept=1, margin_ok=True, greedy=True)
    y = (x / T).astype(np.float32)
    m = float(y.max())
    d = y.astype(np.float64) - m
    keep = np.ones(V, bool)
    margin_ok = True
    if min_p > 0:
        lnm = np.log(min(float(np.float32(min_p)), 1.0))
        keep &= d >= lnm
        gap = np.abs(d - lnm)
        margin_ok &= bool(gap.min() > 1e-5 * max(1.0, abs(lnm)))
    if 0 < k < V:
        kth = np.sort(y)[::-1][k - 1]
        keep &= y >= kth
    w = np.where(keep, np.exp(d), 0.0)
    if np.float32(p) < 1:
        q = float(np.float32(1.0) - np.float32(p))
        idx = np.nonzero(keep)[0]
        order = idx[np.lexsort((idx, y[idx]))]          # ascending value, then ascending index
        c = np.cumsum(w[order]) / w.sum()
        removed = c <= q
        removed[-1] = False
        if np.float32(p) <= 0:
            removed[:] = True
            removed[-1] = False
        else:
            margin_ok &= bool(np.abs(c[:-1] - q).min(initial=1.0) > MARGIN)
        keep[order[removed]] = False
        w = np.where(keep, w, 0.0)
    n_kept = int(keep.sum())
    qe = -np.log(np.asarray(u, np.float64))
    key = np.where(keep, w / qe, -np.inf)
    best = int(np.argmax(key))
    srt = np.sort(key[keep])[::-1]
    if srt.size > 1 and srt[1] >= srt[0] * (1 - MARGIN):
        margin_ok = False
    return dict(token=best, n_kept=n_kept, margin_ok=margin_ok, greedy=False)


def log_softmax(x0):
    x = np.asarray(x0, np.float64)
    m = x.max()
    return x - m - np.log(np.exp(x - m).sum())


def topk_desc(x, k):
    """Top-k ids ordered by (value desc, index asc)."""
    x = np.asarray(x)
    idx = np.arange(x.size)
    order = np.lexsort((idx, -x.astype(np.float64)))
    return order[:k]
