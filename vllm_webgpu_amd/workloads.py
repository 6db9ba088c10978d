"""Synthetic sampling workloads (the five benchmark configurations of this project).

Each configuration draws from ``np.random.default_rng(20261201 + i)`` (i = 1..5) in a fixed
order: logits noise -> spikes / bias permutation -> history -> per-row params -> uniforms.
"N(0, s)" means standard deviation s.  A "Zipf(s) bias over a shuffled permutation" is
``bias[perm[r - 1]] = -s * ln(r)`` for r = 1..V (one permutation shared by the batch).
Uniforms are exact fp32 values in (0, 1): ``rng.integers(1, 2**24) * 2**-24``.

The reference plugin never produces batches (``vllm_webgpu/models/llama.py:182-183`` is
single-sequence) and ships no workloads, so these shapes are the project's own.  ``scale``
shrinks B and V (keeping every other choice) for quick parity tests.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEED_BASE = 20261201


@dataclass
class Workload:
    name: str
    logits: np.ndarray                 # [B, V] float32, uint16 bf16 bit patterns, or float16
    dtype: str                         # "f32" | "bf16" | "f16"
    temperature: np.ndarray            # [B] f32
    top_k: np.ndarray                  # [B] i32 (0 = off)
    top_p: np.ndarray                  # [B] f32 (1 = off)
    min_p: np.ndarray                  # [B] f32 (0 = off)
    repetition: np.ndarray             # [B] f32
    presence: np.ndarray               # [B] f32
    frequency: np.ndarray              # [B] f32
    output_ids: np.ndarray | None      # [B, H] int32 prior output tokens
    uniforms: np.ndarray | None        # [B, V] f32 in (0, 1)
    num_logprobs: int | None = None
    return_probs: bool = False
    extra: dict = field(default_factory=dict)

    @property
    def shape(self):
        return self.logits.shape

    def logits_f32(self) -> np.ndarray:
        if self.dtype == "bf16":
            return (self.logits.astype(np.uint32) << 16).view(np.float32)
        if self.dtype == "f16":
            return self.logits.astype(np.float32)  # exact
        return self.logits


def _uniforms(rng, shape):
    return (rng.integers(1, 2 ** 24, size=shape, dtype=np.int64).astype(np.float32)
            * np.float32(2.0 ** -24))


def _zipf_bias(rng, V, s):
    perm = rng.permutation(V)
    bias = np.empty(V, np.float32)
    bias[perm] = (-s * np.log(np.arange(1, V + 1, dtype=np.float64))).astype(np.float32)
    return bias


def _bf16_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _full(B, v, dt):
    return np.full(B, v, dt)


def config(i: int, scale: float = 1.0) -> Workload:
    """Builds configuration ``i`` (1..5); ``scale`` < 1 shrinks B and V for tests."""
    rng = np.random.default_rng(SEED_BASE + i)

    def dims(B, V):
        if scale >= 1.0:
            return B, V
        return max(1, int(round(B * scale))), max(64, int(round(V * scale)) // 8 * 8)

    if i == 1:
        B, V = dims(1, 32000)
        x = rng.normal(0.0, 2.0, size=(B, V)).astype(np.float32)
        for b in range(B):
            idx = rng.choice(V, size=5, replace=False)
            x[b, idx] += np.float32(8.0)
        return Workload("C1 greedy + T=1 softmax", x, "f32", _full(B, 0.0, np.float32),
                        _full(B, 0, np.int32), _full(B, 1.0, np.float32), _full(B, 0.0, np.float32),
                        _full(B, 1.0, np.float32), _full(B, 0.0, np.float32),
                        _full(B, 0.0, np.float32), None, None, return_probs=True)
    if i == 2:
        B, V = dims(64, 32000)
        x = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
        x += _zipf_bias(rng, V, 1.1)[None, :]
        u = _uniforms(rng, (B, V))
        return Workload("C2 T=0.8 k=50 p=0.9", x, "f32", _full(B, 0.8, np.float32),
                        _full(B, 50, np.int32), _full(B, 0.9, np.float32), _full(B, 0.0, np.float32),
                        _full(B, 1.0, np.float32), _full(B, 0.0, np.float32),
                        _full(B, 0.0, np.float32), None, u)
    if i == 3:
        B, V = dims(256, 128256)
        x = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
        H = 512 if scale >= 1.0 else max(8, int(512 * scale))
        hist = rng.integers(0, V, size=(B, H), dtype=np.int64).astype(np.int32)
        u = _uniforms(rng, (B, V))
        return Workload("C3 penalties + T=0.7 k=50 p=0.9", x, "f32", _full(B, 0.7, np.float32),
                        _full(B, 50, np.int32), _full(B, 0.9, np.float32), _full(B, 0.0, np.float32),
                        _full(B, 1.1, np.float32), _full(B, 0.5, np.float32),
                        _full(B, 0.3, np.float32), hist, u)
    if i == 4:
        B, V = dims(512, 262144)
        x = rng.normal(0.0, 4.0, size=(B, V)).astype(np.float32)
        for b in range(B):
            idx = rng.choice(V, size=10, replace=False)
            x[b, idx] += np.float32(10.0)
        T = rng.uniform(0.0, 1.5, size=B).astype(np.float32)
        greedy = rng.permutation(B)[: B // 8]
        T[greedy] = 0.0
        k = rng.choice(np.array([0, 20, 100], np.int32), size=B).astype(np.int32)
        p = rng.uniform(0.5, 1.0, size=B).astype(np.float32)
        mp = rng.choice(np.array([0.0, 0.05], np.float32), size=B).astype(np.float32)
        u = _uniforms(rng, (B, V))
        return Workload("C4 heterogeneous bf16", _bf16_bits(x), "bf16", T, k, p, mp,
                        _full(B, 1.0, np.float32), _full(B, 0.0, np.float32),
                        _full(B, 0.0, np.float32), None, u)
    if i == 5:
        B, V = dims(1024, 151936)
        x = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
        x += _zipf_bias(rng, V, 1.2)[None, :]
        u = _uniforms(rng, (B, V))
        return Workload("C5 p=0.95 + top-20 logprobs", x, "f32", _full(B, 1.0, np.float32),
                        _full(B, 0, np.int32), _full(B, 0.95, np.float32), _full(B, 0.0, np.float32),
                        _full(B, 1.0, np.float32), _full(B, 0.0, np.float32),
                        _full(B, 0.0, np.float32), None, u, num_logprobs=20)
    raise ValueError(f"unknown config {i}")


def token_state_table(B: int, V: int, prompt_ids: np.ndarray | None = None,
                      output_ids: np.ndarray | None = None) -> np.ndarray:
    """uint32 [B, V] token-state words from padded id lists: bit 31 set for prompt tokens, the
    low bits counting output occurrences (ids outside [0, V) are padding)."""
    st = np.zeros((B, V), np.uint32)
    for ids, prompt in ((prompt_ids, True), (output_ids, False)):
        if ids is None:
            continue
        ok = (ids >= 0) & (ids < V)
        rows = np.broadcast_to(np.arange(B)[:, None], ids.shape)[ok]
        t = ids[ok].astype(np.int64)
        if prompt:
            np.bitwise_or.at(st, (rows, t), np.uint32(0x80000000))
        else:
            np.add.at(st, (rows, t), np.uint32(1))
    return st


def long_history(w: Workload, n_prompt: int = 4096, n_output: int = 1024):
    """C3's rows with a longer history: ``n_prompt`` prompt ids and ``n_output`` output ids per
    row, uniform over V from ``default_rng(SEED_BASE + 30)`` (the first ``H`` output ids are the
    workload's own history)."""
    B, V = w.shape
    rng = np.random.default_rng(SEED_BASE + 30)
    prompt = rng.integers(0, V, size=(B, n_prompt), dtype=np.int64).astype(np.int32)
    out = rng.integers(0, V, size=(B, n_output), dtype=np.int64).astype(np.int32)
    if w.output_ids is not None:
        h = min(n_output, w.output_ids.shape[1])
        out[:, :h] = w.output_ids[:, :h]
    return prompt, out


def algorithmic_bytes(w: Workload, n_kept: np.ndarray | None) -> int:
    """Lower-bound HBM bytes for one pass of the sampler over workload ``w``.

    logits once + history ids + uniforms at the survivors only + 32 B of row params +
    outputs (token id, logprob ids/values + rank, returned probabilities).
    """
    B, V = w.shape
    s = 2 if w.dtype == "bf16" else 4
    total = B * V * s + B * 32 + B * 4
    if w.output_ids is not None:
        total += w.output_ids.size * 4
    if w.uniforms is not None and n_kept is not None:
        greedy = ~(w.temperature >= np.float32(1e-5))
        total += int(np.where(greedy, 0, n_kept).sum()) * 4
    if w.num_logprobs is not None:
        total += B * (8 * (w.num_logprobs + 1) + 8)
    if w.return_probs:
        total += B * V * 4
    return int(total)
