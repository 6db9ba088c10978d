"""Golden fixtures (tests/golden/sampler_golden.npz): the oracle must reproduce them exactly on
the CPU, the float64 brute force must agree on every decidable row, and the GPU library must
reproduce them exactly (token ids, flags, survivor counts, logprob ids and ranks; logprob
values within 1e-5 relative)."""
from __future__ import annotations

import numpy as np
import pytest

from tests.common import FLAG_MASK, LP_ATOL, LP_RTOL
from tests.golden import make_golden as G

FIX = G.load()


def test_fixture_covers_the_crafted_cases():
    assert set(FIX) == set(G.cases())
    assert sum(c["logits"].shape[0] for c in FIX.values()) >= 50


@pytest.mark.parametrize("name", sorted(FIX))
def test_oracle_reproduces_fixture(name):
    c = FIX[name]
    e = G.expected(c)
    for k, v in e.items():
        want = c[f"expect_{k}"]
        assert np.array_equal(v, want), (name, k, v, want)


def test_bruteforce_agrees_with_fixture():
    n = 0
    for name, c in FIX.items():
        e = {k[len("expect_"):]: v for k, v in c.items() if k.startswith("expect_")}
        n += G.check_bruteforce(name, c, e)
    assert n >= 40


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(FIX))
def test_gpu_reproduces_fixture(cuda, name):
    import torch

    from vllm_webgpu_amd import ops

    c = FIX[name]
    print(f"golden case {name} shape {c['logits'].shape}", flush=True)
    if int(c["dtype"]) == 1:
        x = torch.from_numpy(c["logits"].view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        x = torch.from_numpy(c["logits"]).to(cuda)
    greedy_all = bool(np.all(~(c["temperature"] >= np.float32(1e-5))))
    L = int(c["num_logprobs"])
    hist = {}
    if c["prompt_ids"].shape[1]:
        hist["prompt_ids"] = torch.from_numpy(c["prompt_ids"])
    if c["output_ids"].shape[1]:
        hist["output_ids"] = torch.from_numpy(c["output_ids"])
    r = ops.sample(x, temperature=None if greedy_all else torch.from_numpy(c["temperature"]),
                   top_k=torch.from_numpy(c["top_k"]), top_p=torch.from_numpy(c["top_p"]),
                   min_p=torch.from_numpy(c["min_p"]),
                   repetition_penalty=torch.from_numpy(c["rep"]),
                   presence_penalty=torch.from_numpy(c["pres"]),
                   frequency_penalty=torch.from_numpy(c["freq"]),
                   uniforms=None if greedy_all else torch.from_numpy(c["uniforms"]).to(cuda),
                   num_logprobs=L if L >= 0 else None, **hist)
    torch.cuda.synchronize()
    assert np.array_equal(r.sampled.cpu().numpy(), c["expect_token"])
    flags = r.flags.cpu().numpy().view(np.uint32) & FLAG_MASK
    assert np.array_equal(flags, c["expect_flags"])
    assert np.array_equal(r.num_kept.cpu().numpy(), c["expect_n_kept"])
    if L >= 0:
        assert np.array_equal(r.logprob_ids.cpu().numpy(), c["expect_lp_ids"])
        assert np.array_equal(r.logprob_ranks.cpu().numpy(), c["expect_ranks"])
        np.testing.assert_allclose(r.logprob_vals.cpu().numpy(), c["expect_lp_vals"],
                                   rtol=LP_RTOL, atol=LP_ATOL)
