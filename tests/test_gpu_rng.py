"""GPU parity of the generated uniforms: the kernel draws each racing token's uniform from
Philox-4x32-10 keyed by a per-row seed and offset (no [B, V] uniform tensor), and must sample
exactly what the oracle samples from the same generator's uniforms (oracle/vws_oracle.c
vwo_philox_uniforms, pinned by the Random123 known-answer vectors in test_oracle_rng.py).

Every path that races is covered: the single-pass kernel (k <= 64 and k > 64), the top-p
stream (narrow and wide rows), the multi-pass kernel (allowed mask, logprobs)."""
import numpy as np
import pytest

from oracle import sampler as O
from tests.cases import _wl
from tests.common import assert_same, oracle_run
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu


def _seeds(B, salt):
    rng = np.random.default_rng(900 + salt)
    seeds = rng.integers(0, 2 ** 63, B, dtype=np.int64)
    offsets = rng.integers(0, 2 ** 40, B, dtype=np.int64)
    return seeds, offsets


def _run_gen(w, cuda, seeds, offsets, num_logprobs=None, allowed=None):
    import torch

    from vllm_webgpu_amd import ops

    if w.dtype == "bf16":
        logits = torch.from_numpy(w.logits.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        logits = torch.from_numpy(w.logits).to(cuda)
    hist = torch.from_numpy(w.output_ids) if w.output_ids is not None else None
    res = ops.sample(logits, temperature=torch.from_numpy(w.temperature),
                     top_k=torch.from_numpy(w.top_k), top_p=torch.from_numpy(w.top_p),
                     min_p=torch.from_numpy(w.min_p),
                     repetition_penalty=torch.from_numpy(w.repetition),
                     presence_penalty=torch.from_numpy(w.presence),
                     frequency_penalty=torch.from_numpy(w.frequency), output_ids=hist,
                     rng_seeds=torch.from_numpy(seeds), rng_offsets=torch.from_numpy(offsets),
                     num_logprobs=num_logprobs,
                     allowed_mask=None if allowed is None else torch.from_numpy(allowed).to(cuda))
    torch.cuda.synchronize()
    out = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
               n_kept=res.num_kept.cpu().numpy())
    if num_logprobs is not None:
        out.update(lp_ids=res.logprob_ids.cpu().numpy(), lp_vals=res.logprob_vals.cpu().numpy(),
                   ranks=res.logprob_ranks.cpu().numpy())
    return out


def _with_generated(w, seeds, offsets):
    w.uniforms = O.philox_uniforms(seeds.view(np.uint64), w.shape[1], offsets.view(np.uint64))
    return w


@pytest.mark.parametrize("cfg,scale,L", [(2, 1.0, None), (3, 0.25, None), (4, 0.1, None),
                                         (5, 0.1, 20), (5, 0.1, None)])
def test_generated_uniforms_configs(cuda, cfg, scale, L):
    w = W.config(cfg, scale)
    w.num_logprobs = L
    B = w.shape[0]
    seeds, offsets = _seeds(B, cfg)
    g = _run_gen(w, cuda, seeds, offsets, num_logprobs=L)
    assert_same(g, oracle_run(_with_generated(w, seeds, offsets), num_logprobs=L), f"C{cfg} gen")


def test_generated_large_k_and_wide_rows(cuda):
    rng = np.random.default_rng(41)
    B, V = 16, 90000
    x = rng.normal(0, 1.5, (B, V)).astype(np.float32)
    k = np.array([0, 0, 0, 0, 100, 200, 256, 65] * 2, np.int32)
    T = np.array([1.4, 1.2, 1.5, 0.9] * 4, np.float32)
    p = np.array([0.999, 0.99, 0.95, 0.995] * 4, np.float32)
    w = _wl("gen wide", x, T, k=k, p=p, seed=41)
    seeds, offsets = _seeds(B, 41)
    g = _run_gen(w, cuda, seeds, offsets)
    assert int(((g["flags"] & 0x800) != 0).sum()) >= 4   # wide rows took the race pass
    assert_same(g, oracle_run(_with_generated(w, seeds, offsets)), w.name)


def test_generated_multi_pass(cuda):
    """A launch with an allowed mask and logprobs: its top-p rows and k > 256 rows take the
    multi-pass kernel (its k = 20 rows the single pass, which masks their candidates)."""
    rng = np.random.default_rng(42)
    B, V = 8, 20000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    w = _wl("gen multi-pass", x, 0.8, k=np.array([0, 20, 300, 0] * 2, np.int32), p=0.9, seed=42)
    allowed_bool = rng.random((B, V)) < 0.7
    words = np.zeros((B, (V + 31) // 32 * 32), np.uint64)
    words[:, :V] = allowed_bool
    bits = (words.reshape(B, -1, 32) << np.arange(32, dtype=np.uint64)).sum(axis=2).astype(np.uint32)
    seeds, offsets = _seeds(B, 42)
    g = _run_gen(w, cuda, seeds, offsets, num_logprobs=3, allowed=bits.view(np.int32))
    w = _with_generated(w, seeds, offsets)
    prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence,
                        w.frequency)
    ref = O.sample(w.logits_f32(), prm, w.uniforms, num_logprobs=3, allowed=bits)
    assert_same(g, ref, w.name)


def test_offsets_and_seeds_change_the_draws(cuda):
    """The same logits with other keys sample other tokens (flat rows: every token races)."""
    B, V = 64, 5000
    x = np.zeros((B, V), np.float32)
    w = _wl("flat", x, 1.0, seed=43)
    seeds, offsets = _seeds(B, 43)
    a = _run_gen(w, cuda, seeds, offsets)["token"]
    b = _run_gen(w, cuda, seeds, offsets + 1)["token"]
    c = _run_gen(w, cuda, seeds + 1, offsets)["token"]
    assert np.array_equal(a, _run_gen(w, cuda, seeds, offsets)["token"])   # deterministic
    assert (a != b).sum() > B // 2 and (a != c).sum() > B // 2
    # flat rows: the winner is the largest uniform of the row
    u = O.philox_uniforms(seeds.view(np.uint64), V, offsets.view(np.uint64))
    assert np.array_equal(a, np.argmax(u, axis=1))


def _run_key(w, cuda, key, num_logprobs=None):
    import torch

    from vllm_webgpu_amd import ops

    if w.dtype == "bf16":
        logits = torch.from_numpy(w.logits.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        logits = torch.from_numpy(w.logits).to(cuda)
    hist = torch.from_numpy(w.output_ids) if w.output_ids is not None else None
    res = ops.sample(logits, temperature=torch.from_numpy(w.temperature),
                     top_k=torch.from_numpy(w.top_k), top_p=torch.from_numpy(w.top_p),
                     min_p=torch.from_numpy(w.min_p),
                     repetition_penalty=torch.from_numpy(w.repetition),
                     presence_penalty=torch.from_numpy(w.presence),
                     frequency_penalty=torch.from_numpy(w.frequency), output_ids=hist,
                     rng_key=key, num_logprobs=num_logprobs)
    torch.cuda.synchronize()
    out = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
               n_kept=res.num_kept.cpu().numpy())
    if num_logprobs is not None:
        out.update(lp_ids=res.logprob_ids.cpu().numpy(), lp_vals=res.logprob_vals.cpu().numpy(),
                   ranks=res.logprob_ranks.cpu().numpy())
    return out


@pytest.mark.parametrize("cfg,scale,L", [(3, 0.25, None), (4, 0.1, None), (5, 0.1, 20)])
def test_launch_key(cuda, cfg, scale, L):
    """One by-value key for the launch: row r draws as with seed key and offset r -- the same
    tokens as those per-row keys passed as arrays, and as the oracle with their uniforms."""
    w = W.config(cfg, scale)
    w.num_logprobs = L
    B = w.shape[0]
    key = 0xC0FFEE1234567 + cfg  # above 2^32: both key words matter
    seeds = np.full(B, key, np.int64)
    offsets = np.arange(B, dtype=np.int64)
    g = _run_key(w, cuda, key, num_logprobs=L)
    assert_same(g, _run_gen(w, cuda, seeds, offsets, num_logprobs=L), f"C{cfg} key vs arrays")
    assert_same(g, oracle_run(_with_generated(w, seeds, offsets), num_logprobs=L), f"C{cfg} key")
