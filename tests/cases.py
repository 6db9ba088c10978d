"""Crafted edge-case workloads shared by the golden-fixture generator and the parity tests.

Each case stresses one rule of the sampler: ties at the argmax and at the k-th value, a top-p
boundary inside a tie group, all-equal rows, greedy rows mixed with random ones, duplicate
history tokens, penalties that raise logits, min-p leaving only the max, unaligned rows,
-inf logits and tiny vocabularies."""
from __future__ import annotations

import numpy as np

from vllm_webgpu_amd.workloads import Workload


def _u(rng, shape):
    return rng.integers(1, 2 ** 24, size=shape, dtype=np.int64).astype(np.float32) * np.float32(2.0 ** -24)


def _wl(name, x, T, k=0, p=1.0, mp=0.0, rep=1.0, pres=0.0, freq=0.0, hist=None, seed=0,
        dtype="f32", u=None, L=None):
    B, V = x.shape
    rng = np.random.default_rng(seed + 7)

    def full(v, dt):
        a = np.asarray(v, dt)
        return np.broadcast_to(a, (B,)).copy() if a.ndim == 0 else a.astype(dt)
    if u is None:
        u = _u(rng, (B, V))
    return Workload(name, x, dtype, full(T, np.float32), full(k, np.int32), full(p, np.float32),
                    full(mp, np.float32), full(rep, np.float32), full(pres, np.float32),
                    full(freq, np.float32), hist, u, num_logprobs=L)


def all_cases():
    cs = []
    rng = np.random.default_rng(11)
    # argmax ties: the max appears several times; the lowest index must win
    x = rng.normal(0, 1, (6, 3000)).astype(np.float32)
    for b in range(6):
        pos = rng.choice(3000, size=b + 2, replace=False)
        x[b, pos] = 9.0
    cs.append(_wl("greedy_ties", x, 0.0, seed=1))
    # the reference's planted known answers (tests/test_kernels_sample.py:13-16,55-58,122-145)
    x = rng.normal(0, 1, (9, 128)).astype(np.float16).astype(np.float32)
    x[0, 77] = 100.0
    for b, t in enumerate(range(0, 128, 16)):
        x[b + 1] = (rng.normal(0, 1, 128) * 0.1).astype(np.float16).astype(np.float32)
        x[b + 1, t] = 50.0
    cs.append(_wl("planted_argmax", x, 0.0, seed=2))
    # all-equal rows: one tie group covers the row; top-p removes the lowest indices
    x = np.full((3, 4096), 1.5, np.float32)
    cs.append(_wl("all_equal_topp", x, 1.0, p=np.array([0.9, 0.5, 0.999], np.float32), seed=3))
    cs.append(_wl("all_equal_topk", x, 1.0, k=np.array([10, 100, 256], np.int32), p=0.7, seed=4))
    # heavy ties at the k-th value (values on a coarse grid)
    x = np.round(rng.normal(0, 2, (8, 5000)) * 2).astype(np.float32) / 2
    cs.append(_wl("grid_ties_topk", x, 0.9, k=np.array([1, 5, 20, 50, 100, 200, 256, 7], np.int32),
                  p=0.8, seed=5))
    cs.append(_wl("grid_ties_topp", x, 0.9, p=np.array([0.3, 0.5, 0.6, 0.7, 0.8, 0.9, 0.95, 0.99], np.float32), seed=6))
    # min-p keeps only the max (min_p = 1), single survivor by top-k = 1
    x = rng.normal(0, 3, (4, 2000)).astype(np.float32)
    cs.append(_wl("minp_one", x, 0.8, mp=1.0, seed=7))
    cs.append(_wl("topk_one", x, 0.8, k=1, p=0.9, seed=8))
    cs.append(_wl("minp_only", x, 1.3, mp=np.array([0.01, 0.05, 0.1, 0.5], np.float32), seed=9))
    # top-p extremes: tiny p, p = 0, p = 1 (off)
    cs.append(_wl("topp_extremes", x, 0.7, p=np.array([1e-9, 0.0, 1.0, 0.5], np.float32), seed=10))
    # greedy rows mixed with random rows
    x = rng.normal(0, 3, (8, 3000)).astype(np.float32)
    T = np.array([0.0, 0.7, 1e-6, 1.0, 0.0, 1.5, 1e-5, 0.9], np.float32)
    cs.append(_wl("greedy_mixed", x, T, k=np.array([0, 50, 0, 20, 5, 0, 10, 0], np.int32),
                  p=np.array([1.0, 0.9, 0.8, 1.0, 0.5, 0.95, 0.9, 0.6], np.float32), seed=11))
    # large k (beyond the single-pass kernel), top-k off with top-p and min-p
    x = rng.normal(0, 3, (4, 6000)).astype(np.float32)
    cs.append(_wl("large_k", x, 1.0, k=np.array([300, 1000, 5000, 5999], np.int32), p=0.95, seed=12))
    cs.append(_wl("topp_minp_general", x, 0.8, p=0.9, mp=np.array([0.0, 0.02, 0.1, 0.0], np.float32), seed=13))
    # penalties: duplicates in the history, prompt tokens, penalties that raise logits
    x = rng.normal(0, 3, (6, 4000)).astype(np.float32)
    hist = rng.integers(0, 4000, (6, 64)).astype(np.int32)
    hist[:, :16] = hist[:, :1]           # one token repeated 16 times
    hist[:, 60:] = 4000                  # vLLM-style padding (= V)
    top = np.argsort(-x, axis=1)[:, :8].astype(np.int32)
    hist[:, 16:24] = top                 # penalise the current top tokens
    cs.append(_wl("penalties_topk", x, 0.7, k=50, p=0.9, rep=1.3, pres=0.5, freq=0.4, hist=hist, seed=14))
    cs.append(_wl("penalties_raise", x, 0.7, k=50, p=0.9,
                  rep=np.array([0.8, 0.5, 1.0, 2.0, 0.9, 1.1], np.float32),
                  pres=np.array([-0.5, 0.0, -2.0, 0.5, 0.0, -1.0], np.float32),
                  freq=np.array([-0.3, -1.0, 0.0, 0.2, -0.1, 0.0], np.float32), hist=hist, seed=15))
    cs.append(_wl("penalties_greedy", x, 0.0, rep=1.5, pres=0.7, freq=0.2, hist=hist, seed=16))
    cs.append(_wl("penalties_general", x, 0.9, p=0.8, rep=1.2, pres=0.3, freq=0.1, hist=hist, seed=17))
    # unaligned rows (odd V) and tiny vocabularies
    x = rng.normal(0, 2, (5, 4099)).astype(np.float32)
    cs.append(_wl("unaligned", x, 0.9, k=np.array([0, 10, 40, 0, 3], np.int32), p=0.9, seed=18))
    for V in (1, 2, 3, 7):
        x = rng.normal(0, 2, (3, V)).astype(np.float32)
        cs.append(_wl(f"tiny_V{V}", x, np.array([0.0, 1.0, 0.5], np.float32), k=np.array([0, 1, 2], np.int32),
                      p=0.9, seed=19 + V))
    # -inf logits (masked tokens) and rows that are almost all -inf
    x = rng.normal(0, 2, (4, 3000)).astype(np.float32)
    x[:, ::3] = -np.inf
    x[3, :] = -np.inf
    x[3, 1234] = 0.5
    cs.append(_wl("neg_inf", x, 0.8, k=np.array([0, 20, 0, 5], np.int32), p=0.9, seed=30))
    # uniforms at the ends of (0, 1)
    x = rng.normal(0, 1, (4, 2048)).astype(np.float32)
    u = np.full((4, 2048), 0.5, np.float32)
    u[0] = np.float32(1 - 2.0 ** -24)
    u[1] = np.float32(2.0 ** -24)
    u[2, ::2] = np.float32(1 - 2.0 ** -24)
    cs.append(_wl("uniform_ends", x, 1.0, k=np.array([20, 20, 0, 0], np.int32), p=0.9, seed=31, u=u))
    # logprobs on mixed rows (greedy, top-k, top-p) incl. penalties
    x = rng.normal(0, 3, (6, 5000)).astype(np.float32)
    hist = rng.integers(0, 5000, (6, 32)).astype(np.int32)
    cs.append(_wl("logprobs_mixed", x, np.array([0.0, 1.0, 0.7, 1.0, 0.0, 1.2], np.float32),
                  k=np.array([0, 0, 40, 0, 0, 100], np.int32),
                  p=np.array([1.0, 0.95, 0.9, 0.5, 1.0, 1.0], np.float32), rep=1.1, pres=0.2,
                  hist=hist, seed=32, L=5))
    cs.append(_wl("logprobs_plain", x, 1.0, p=0.95, seed=33, L=20))
    # bf16 rows (exact widening), heavy ties
    xb = rng.normal(0, 4, (6, 8192)).astype(np.float32)
    from vllm_webgpu_amd.workloads import _bf16_bits
    bits = _bf16_bits(xb)
    cs.append(_wl("bf16_mixed", bits, np.array([0.0, 1.0, 0.5, 1.2, 0.8, 1.0], np.float32),
                  k=np.array([0, 20, 100, 0, 0, 7], np.int32),
                  p=np.array([1.0, 0.9, 0.7, 0.6, 1.0, 0.95], np.float32),
                  mp=np.array([0.0, 0.05, 0.0, 0.05, 0.1, 0.0], np.float32), dtype="bf16", seed=34))
    return cs
