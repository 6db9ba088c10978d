"""The device sampler draws from the reference CLI sampler's distribution
(``run_inference.py:383-390``: ``p = softmax(x / T)``, then ``np.random.choice(V, p=p)``): many
rows with the same logits and independent uniforms, token frequencies against the float64
probabilities, with and without top-k truncation, by a chi-square test."""
import numpy as np
import pytest
import torch
from scipy import stats

from vllm_webgpu_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("k", [0, 6])     # 0: top-k off (multi-pass path); 6: single-pass path
def test_race_matches_softmax(cuda, k):
    V, B, T = 16, 1 << 16, 0.8
    x = np.linspace(-2.0, 2.5, V).astype(np.float32)[np.random.default_rng(1).permutation(V)]
    rng = np.random.default_rng(2 + k)
    u = (rng.integers(1, 2 ** 24, (B, V)) * 2.0 ** -24).astype(np.float32)
    logits = torch.from_numpy(np.tile(x, (B, 1))).to(cuda)
    res = ops.sample(logits, temperature=T, top_k=k, uniforms=torch.from_numpy(u).to(cuda))
    tok = res.sampled.cpu().numpy()
    y = x.astype(np.float64) / T
    keep = np.ones(V, bool)
    if k:
        keep = y >= np.sort(y)[::-1][k - 1]
    p = np.where(keep, np.exp(y - y.max()), 0.0)
    p /= p.sum()
    counts = np.bincount(tok, minlength=V)
    assert counts[~keep].sum() == 0
    chi2, pval = stats.chisquare(counts[keep], B * p[keep])
    assert pval > 1e-4, (chi2, pval, counts, B * p)
