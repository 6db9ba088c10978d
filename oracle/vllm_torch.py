"""vLLM-v1 Sampler restated with torch CPU tensor ops -- TEST INFRASTRUCTURE ONLY.

The reference plugin leaves non-greedy sampling to "vLLM's sampler [which] runs on CPU"
(``docs/superpowers/specs/2026-06-29-vllm-webgpu-design.md:451``; vLLM is a dependency,
``pyproject.toml:10``, not vendored).  This module writes that sampler's op sequence down with
torch CPU tensors, in the order vLLM-v1 applies it:

1. raw logprobs = log_softmax(logits) (fp32) when logprobs are requested;
2. penalties from bin counts over ``[B, V+1]`` (pad id V): repetition on prompt|output tokens
   (``x > 0 ? x * (1/r) : x * r``), then ``x -= f * count``, then ``x -= p * (count > 0)``;
3. greedy result = argmax of the penalised logits (used where ``T < 1e-5``);
4. temperature ``x / T`` (T replaced by 1 on greedy rows);
5. min-p: mask ``softmax(x) < max(softmax(x)) * min_p``;
6. top-k / top-p on an ascending stable sort: mask values below the k-th largest, then mask
   the prefix whose cumulative softmax mass is ``<= 1 - p`` (always keeping the largest);
7. exponential race ``argmax(softmax(x) / q)`` with ``q = -ln(u)`` from caller uniforms;
8. logprobs: top-L of the raw logprobs, the sampled token's logprob and its rank
   ``#{j : lp_j >= lp_sampled}``.

It is the CPU baseline that bench.py times, and a second, independent statement of the
semantics: token ids must agree with ``oracle/sampler.py`` on every row that is not a near
tie (tests/test_oracle_vs_vllm_torch.py).  ``compute_dtype=torch.float64`` gives a
higher-precision variant for margin analysis.
"""
from __future__ import annotations

import torch

SAMPLING_EPS = 1e-5


def bin_counts(tokens: torch.Tensor, V: int) -> torch.Tensor:
    """Counts of each id in [0, V) per row; ids outside [0, V) (padding) are ignored."""
    B = tokens.shape[0]
    t = tokens.to(torch.int64).clone()
    t[(t < 0) | (t >= V)] = V
    counts = torch.zeros((B, V + 1), dtype=torch.int64)
    counts.scatter_add_(1, t, torch.ones_like(t))
    return counts[:, :V]


def apply_penalties(x, prompt_ids, output_ids, rep, pres, freq):
    B, V = x.shape
    prompt_mask = (bin_counts(prompt_ids, V) > 0) if prompt_ids is not None else torch.zeros_like(x, dtype=torch.bool)
    out_counts = bin_counts(output_ids, V) if output_ids is not None else torch.zeros((B, V), dtype=torch.int64)
    out_mask = out_counts > 0
    pen = torch.where(prompt_mask | out_mask, rep[:, None].expand(B, V), torch.ones_like(x))
    scaling = torch.where(x > 0, 1.0 / pen, pen)
    x = x * scaling
    x = x - freq[:, None] * out_counts.to(x.dtype)
    x = x - pres[:, None] * out_mask.to(x.dtype)
    return x


def sample(logits: torch.Tensor, temperature, top_k, top_p, min_p, repetition, presence,
           frequency, uniforms: torch.Tensor, prompt_ids=None, output_ids=None,
           num_logprobs: int | None = None, compute_dtype=torch.float32) -> dict:
    """All per-row parameters are 1-D CPU tensors of length B; logits [B, V] (any float dtype)."""
    B, V = logits.shape
    out = {}
    if num_logprobs is not None:
        raw = logits.to(torch.float32).log_softmax(dim=-1)
    x = logits.to(torch.float32)
    has_pen = prompt_ids is not None or output_ids is not None
    if has_pen:
        x = apply_penalties(x, prompt_ids, output_ids, repetition.float(), presence.float(),
                            frequency.float())
    greedy = x.argmax(dim=-1)
    x = x.to(compute_dtype)
    T = temperature.to(compute_dtype)
    is_greedy = ~(temperature >= SAMPLING_EPS)
    T = torch.where(is_greedy, torch.ones_like(T), T)
    x = x / T[:, None]
    mp = min_p.to(compute_dtype)
    if bool((mp > 0).any()):
        probs = x.softmax(dim=-1)
        maxp = probs.amax(dim=-1, keepdim=True)
        x = x.masked_fill(probs < maxp * mp[:, None], float("-inf"))
    xs, order = x.sort(dim=-1, descending=False, stable=True)
    k = top_k.to(torch.int64)
    k_on = (k > 0) & (k < V)
    kk = torch.where(k_on, k, torch.full_like(k, V))
    kth = xs.gather(1, (V - kk).unsqueeze(1))
    xs = xs.masked_fill(xs < kth, float("-inf"))
    p = top_p.to(compute_dtype)
    probs_sort = xs.softmax(dim=-1)
    csum = probs_sort.cumsum(dim=-1)
    pmask = csum <= (1 - p)[:, None]
    pmask[:, -1] = False
    xs = xs.masked_fill(pmask, float("-inf"))
    x = torch.empty_like(xs).scatter_(1, order, xs)
    probs = x.softmax(dim=-1)
    q = -torch.log(uniforms.to(compute_dtype))
    race = (probs / q).argmax(dim=-1)
    token = torch.where(is_greedy, greedy, race)
    out["token"] = token.to(torch.int32)
    out["n_kept"] = torch.where(is_greedy, torch.ones_like(token), (probs > 0).sum(-1))
    if num_logprobs is not None:
        lp_tok = raw.gather(1, token.unsqueeze(1))
        rank = (raw >= lp_tok).sum(-1)
        ids = [token.unsqueeze(1).to(torch.int32)]
        vals = [lp_tok]
        if num_logprobs > 0:
            tv, ti = raw.topk(num_logprobs, dim=-1)
            ids.append(ti.to(torch.int32))
            vals.append(tv)
        out["lp_ids"] = torch.cat(ids, 1)
        out["lp_vals"] = torch.cat(vals, 1)
        out["ranks"] = rank.to(torch.int32)
    return out
