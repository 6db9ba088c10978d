"""Writes tests/golden/sampler_golden.npz: small crafted sampling cases with their expected
outputs (token ids, flags, survivor counts, logprobs).

Inputs are seeded and crafted to hit one rule each (shapes 8x64, 4x1000, 2x4096 bf16 and a
few tiny rows): ties at the argmax and at the k-th value, a top-p boundary inside a tie group,
+0/-0, all-equal rows, a single survivor, greedy rows mixed with sampled rows, duplicate and
padded history ids, min-p leaving only the max, -inf logits, and the reference's own planted
known answers (``tests/test_kernels_sample.py:13-16,55-58,122-145``).

Expected outputs come from the CPU oracle (``oracle/sampler.py``); before writing, every row
whose float64 brute force (``tests/bruteforce.py``) is decidable must agree with it, so a
fixture never freezes an oracle mistake.  Run from the repository root:

    python -m tests.golden.make_golden
"""
from __future__ import annotations

import os

import numpy as np

from oracle import sampler as O
from tests import bruteforce as BF

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sampler_golden.npz")
FIELDS = ("logits", "temperature", "top_k", "top_p", "min_p", "rep", "pres", "freq", "uniforms",
          "prompt_ids", "output_ids")


def _u(rng, shape):
    return (rng.integers(1, 2 ** 24, size=shape) * 2.0 ** -24).astype(np.float32)


def _case(x, T, k=0, p=1.0, mp=0.0, rep=1.0, pres=0.0, freq=0.0, prompt=None, output=None,
          seed=0, bf16=False, L=-1):
    B, V = x.shape
    rng = np.random.default_rng(1000 + seed)

    def row(v, dt):
        return np.broadcast_to(np.asarray(v, dt), (B,)).copy()
    c = dict(logits=O.f32_to_bf16_bits(x) if bf16 else x.astype(np.float32),
             temperature=row(T, np.float32), top_k=row(k, np.int32), top_p=row(p, np.float32),
             min_p=row(mp, np.float32), rep=row(rep, np.float32), pres=row(pres, np.float32),
             freq=row(freq, np.float32), uniforms=_u(rng, (B, V)),
             prompt_ids=np.zeros((B, 0), np.int32) if prompt is None else prompt.astype(np.int32),
             output_ids=np.zeros((B, 0), np.int32) if output is None else output.astype(np.int32),
             dtype=np.array(1 if bf16 else 0, np.int32), num_logprobs=np.array(L, np.int32))
    return c


def cases() -> dict:
    rng = np.random.default_rng(20261201)
    cs = {}
    # reference known answers: 100.0 at 77 (V=128); unique max 50.0 at 0, 16, ..., 112
    x = rng.normal(0, 1, (9, 128)).astype(np.float16).astype(np.float32)
    x[0, 77] = 100.0
    for b, t in enumerate(range(0, 128, 16)):
        x[b + 1] = 0.1 * rng.normal(0, 1, 128).astype(np.float16).astype(np.float32)
        x[b + 1, t] = 50.0
    cs["kat_argmax"] = _case(x, 0.0, seed=1)
    # greedy ties on fp16-representable values, 8 x 64
    x = rng.integers(-4, 5, (8, 64)).astype(np.float32) * np.float32(0.5)
    cs["greedy_ties_8x64"] = _case(x, 0.0, seed=2)
    # mixed per-row parameters with penalties and duplicate / padded history, 8 x 64
    x = rng.normal(0, 2, (8, 64)).astype(np.float16).astype(np.float32)
    hist = rng.integers(0, 65, (8, 12))                      # 64 = padding
    hist[:, :3] = hist[:, 3:6]                               # duplicates
    prompt = rng.integers(0, 64, (8, 5))
    cs["mixed_8x64"] = _case(
        x, np.array([0.0, 0.5, 0.7, 1.0, 1.3, 0.9, 2.0, 1e-6], np.float32),
        k=np.array([0, 5, 1, 10, 64, 3, 0, 7], np.int32),
        p=np.array([1.0, 0.9, 0.5, 0.3, 0.95, 1.0, 0.8, 0.1], np.float32),
        mp=np.array([0.0, 0.0, 0.1, 0.0, 0.05, 0.3, 0.0, 0.0], np.float32),
        rep=np.array([1.0, 1.1, 1.3, 0.8, 1.0, 1.1, 1.2, 1.5], np.float32),
        pres=np.array([0.0, 0.5, 0.0, 0.2, 0.0, 0.5, 1.0, 0.0], np.float32),
        freq=np.array([0.0, 0.3, 0.1, 0.0, 0.0, 0.3, 0.5, 0.0], np.float32),
        prompt=prompt, output=hist, seed=3)
    # penalties + top-k + top-p at V=1000
    x = rng.normal(0, 3, (4, 1000)).astype(np.float32)
    hist = rng.integers(0, 1000, (4, 40))
    hist[:, :8] = hist[:, 8:16]
    cs["penalties_4x1000"] = _case(x, 0.7, k=np.array([50, 0, 256, 20], np.int32), p=0.9,
                                   rep=1.1, pres=0.5, freq=0.3, output=hist, seed=4)
    # bf16 logits, top-k and untruncated top-p rows
    x = rng.normal(0, 4, (2, 4096)).astype(np.float32)
    x[:, rng.choice(4096, 6, replace=False)] += 10
    cs["bf16_2x4096"] = _case(x, 0.8, k=np.array([50, 0], np.int32), p=0.9, seed=5, bf16=True)
    # all-equal rows: top-p removes the lowest indices of one tie group; top-k keeps the group
    x = np.full((4, 256), -1.25, np.float32)
    cs["all_equal_4x256"] = _case(x, 1.0, k=np.array([0, 10, 0, 1], np.int32),
                                  p=np.array([0.5, 1.0, 0.75, 0.2], np.float32), seed=6)
    # top-p boundary inside a tie group (coarse grid of values)
    x = np.round(rng.normal(0, 1.5, (6, 500)) * 2).astype(np.float32) / 2
    cs["grid_ties_6x500"] = _case(x, 1.0, k=np.array([0, 0, 5, 20, 0, 50], np.int32),
                                  p=np.array([0.5, 0.8, 0.9, 0.6, 0.95, 0.7], np.float32), seed=7)
    # +0 / -0 as the row maximum: equal keys, the lowest index wins
    x = np.full((3, 64), -2.0, np.float32)
    x[0, [9, 3]] = [0.0, -0.0]
    x[1, [4, 40]] = [-0.0, 0.0]
    x[2, [1, 2]] = [-0.0, -0.0]
    cs["signed_zero_3x64"] = _case(x, np.array([0.0, 0.0, 1.0], np.float32),
                                   k=np.array([0, 0, 2], np.int32), seed=8)
    # min-p = 1 and top-k = 1: single survivor
    x = rng.normal(0, 3, (4, 300)).astype(np.float32)
    cs["single_survivor_4x300"] = _case(x, 0.8, k=np.array([0, 1, 0, 1], np.int32),
                                        mp=np.array([1.0, 0.0, 1.0, 0.5], np.float32), seed=9)
    # -inf logits (masked vocabulary) with top-p and top-k
    x = rng.normal(0, 2, (3, 200)).astype(np.float32)
    x[:, 50:150] = -np.inf
    cs["neg_inf_3x200"] = _case(x, np.array([0.0, 1.0, 0.6], np.float32),
                                k=np.array([0, 0, 30], np.int32), p=0.9, seed=10)
    # raw top-L logprobs with ties among the top values
    x = rng.normal(0, 3, (4, 1000)).astype(np.float32)
    x[0, [5, 600, 900]] = x[0].max() + 1
    cs["logprobs_4x1000"] = _case(x, np.array([1.0, 0.0, 0.7, 1.0], np.float32),
                                  p=np.array([0.95, 1.0, 0.9, 1.0], np.float32), seed=11, L=5)
    return cs


def expected(c: dict) -> dict:
    x = c["logits"]
    if int(c["dtype"]) == 1:
        x = O.bf16_bits_to_f32(x)
    B = x.shape[0]
    prm = O.make_params(B, c["temperature"], c["top_k"], c["top_p"], c["min_p"], c["rep"],
                        c["pres"], c["freq"])
    L = int(c["num_logprobs"])
    r = O.sample(x, prm, c["uniforms"],
                 prompt_ids=c["prompt_ids"] if c["prompt_ids"].shape[1] else None,
                 output_ids=c["output_ids"] if c["output_ids"].shape[1] else None,
                 num_logprobs=L if L >= 0 else None)
    out = dict(token=r["token"], flags=(r["flags"] & 0xFF).astype(np.uint32), n_kept=r["n_kept"])
    if L >= 0:
        out.update(lp_ids=r["lp_ids"], lp_vals=r["lp_vals"], ranks=r["ranks"])
    return out


def check_bruteforce(name: str, c: dict, e: dict) -> int:
    """Asserts agreement with the float64 brute force on decidable rows; returns rows checked."""
    x = c["logits"]
    if int(c["dtype"]) == 1:
        x = O.bf16_bits_to_f32(x)
    n = 0
    for b in range(x.shape[0]):
        if not np.isfinite(x[b]).any() or np.isnan(x[b]).any():
            continue
        if not np.isfinite(np.max(x[b])):
            continue
        w = BF.sample_row(x[b], c["temperature"][b], int(c["top_k"][b]), c["top_p"][b],
                          c["min_p"][b], c["rep"][b], c["pres"][b], c["freq"][b],
                          c["uniforms"][b], prompt=c["prompt_ids"][b], output=c["output_ids"][b])
        if not w["margin_ok"] or (e["flags"][b] & 0x3):
            continue
        assert e["token"][b] == w["token"], (name, b, e["token"][b], w["token"])
        assert e["n_kept"][b] == w["n_kept"], (name, b, e["n_kept"][b], w["n_kept"])
        n += 1
    return n


def load(path: str = OUT) -> dict:
    """Returns {case: {field: array}} from the fixture file (no pickles)."""
    z = np.load(path, allow_pickle=False)
    out: dict = {}
    for key in z.files:
        case, field = key.split("/", 1)
        out.setdefault(case, {})[field] = z[key]
    return out


def main():
    flat = {}
    for name, c in cases().items():
        e = expected(c)
        check_bruteforce(name, c, e)
        for k, v in c.items():
            flat[f"{name}/{k}"] = v
        for k, v in e.items():
            flat[f"{name}/expect_{k}"] = v
    np.savez_compressed(OUT, **flat)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(flat)} arrays)")


if __name__ == "__main__":
    main()
