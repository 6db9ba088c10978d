"""GPU parity of the vLLM-v1 front end: ``Sampler.forward`` and the model runner's
``execute_model`` / ``sample_tokens`` loop against the CPU oracle on the same inputs.

Every random row is seeded, so the per-row keys the sampler draws (the race's uniforms are
generated from them in the kernel) can be redrawn here from generators with the same seeds, and
the oracle's copy of the generator turns them into the same uniforms; tokens must then agree bit for bit and
raw logprobs within rtol 1e-5."""
from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from oracle import sampler as O
from vllm_webgpu_amd import workloads as W
from vllm_webgpu_amd.v1.model_runner import ROCmModelRunner
from vllm_webgpu_amd.v1.sample.metadata import SamplingMetadata
from vllm_webgpu_amd.v1.sample.sampler import KeyStream, Sampler, draw_seeds

pytestmark = pytest.mark.gpu


def _gens(B, dev, base):
    return {i: torch.Generator(device=dev).manual_seed(base + i) for i in range(B)}


def _metadata(w, dev, gens, num_logprobs):
    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    hist = t(w.output_ids) if w.output_ids is not None else None
    no_pen = hist is None
    greedy = ~(w.temperature >= np.float32(1e-5))
    return SamplingMetadata(
        temperature=None if greedy.all() else t(w.temperature), all_greedy=bool(greedy.all()),
        all_random=not greedy.any(), top_p=t(w.top_p), top_k=t(w.top_k), generators=gens,
        max_num_logprobs=num_logprobs, no_penalties=no_pen, prompt_token_ids=None,
        frequency_penalties=t(w.frequency), presence_penalties=t(w.presence),
        repetition_penalties=t(w.repetition), output_token_ids=[], min_p=t(w.min_p),
        output_token_ids_tensor=hist)


@pytest.mark.parametrize("cfg,scale,L,cap", [(2, 0.25, None, None), (3, 0.05, None, None),
                                             (4, 0.05, None, None), (5, 0.05, 20, None),
                                             (3, 0.05, None, 30.0), (5, 0.05, 20, 30.0)])
def test_sampler_forward_matches_oracle(cuda, cfg, scale, L, cap):
    w = W.config(cfg, scale=scale)
    B, V = w.shape
    if w.dtype == "bf16":
        logits = torch.from_numpy(w.logits.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        logits = torch.from_numpy(w.logits).to(cuda)
    out = Sampler(logit_softcap=cap)(logits, _metadata(w, cuda, _gens(B, cuda, 7000), L))
    u = O.philox_uniforms(draw_seeds(B, _gens(B, cuda, 7000), cuda).cpu().numpy(), V)
    prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence,
                        w.frequency)
    ref = O.sample(w.logits_f32(), prm, u, output_ids=w.output_ids, num_logprobs=L, softcap=cap)
    tok = out.sampled_token_ids.cpu().numpy()
    assert tok.shape == (B, 1) and tok.dtype == np.int32
    bad = np.nonzero(tok[:, 0] != ref["token"])[0]
    assert bad.size == 0, f"rows {bad[:8]}: gpu {tok[bad[:8], 0]} oracle {ref['token'][bad[:8]]}"
    if L is None:
        assert out.logprobs_tensors is None
    else:
        lp = out.logprobs_tensors
        np.testing.assert_array_equal(lp.logprob_token_ids.cpu().numpy(), ref["lp_ids"])
        np.testing.assert_array_equal(lp.selected_token_ranks.cpu().numpy(), ref["ranks"])
        np.testing.assert_allclose(lp.logprobs.cpu().numpy(), ref["lp_vals"], rtol=1e-5, atol=1e-6)


class _FakeModel:
    """Deterministic logits per step (seeded), kept for the oracle check."""

    def __init__(self, V, dev):
        self.vocab_size, self.dev, self.step, self.history = V, dev, 0, []

    def forward(self, input_ids, positions, scheduler_output):
        rng = np.random.default_rng(900 + self.step)
        x = rng.normal(0.0, 3.0, (input_ids.shape[0], self.vocab_size)).astype(np.float32)
        # make recent inputs likely again so the penalties matter
        ids = input_ids.cpu().numpy()
        x[np.arange(len(ids)), ids % self.vocab_size] += 6.0
        self.step += 1
        self.history.append(x)
        return torch.from_numpy(x).to(self.dev)


def _sp(**kw):
    base = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0,
                presence_penalty=0.0, frequency_penalty=0.0, seed=None, logprobs=None)
    base.update(kw)
    return NS(**base)


@pytest.mark.parametrize("token_state", [True, False])
def test_runner_steps_match_oracle(cuda, token_state):
    """Six runner steps of mixed requests against the oracle on the id lists; the runner keeps
    the penalties' history as its device token-state table or as gathered id lists."""
    V = 4096
    model = _FakeModel(V, cuda)
    runner = ROCmModelRunner(None, cuda, model, max_num_reqs=8, max_prompt_len=64,
                             max_output_len=32, token_state=token_state)
    params = {
        "g": _sp(temperature=0.0, repetition_penalty=1.5),
        "k": _sp(temperature=0.8, top_k=20, seed=11, presence_penalty=0.4),
        "p": _sp(temperature=1.0, top_p=0.9, repetition_penalty=1.3, presence_penalty=0.2,
                 frequency_penalty=0.1, seed=12),
        "m": _sp(temperature=0.6, min_p=0.1, logprobs=5, seed=13, frequency_penalty=0.5),
        "late": _sp(temperature=0.9, top_k=50, top_p=0.8, seed=14, repetition_penalty=1.2),
    }
    prompts = {"g": [1, 2, 3], "k": [5, 5, 9, 4000], "p": [17], "m": [2, 3, 5, 7, 11, 13],
               "late": [100, 200]}
    mirror = {r: KeyStream(params[r].seed)
              for r in params if params[r].seed is not None}
    outputs = {r: [] for r in params}
    active = []
    for step in range(6):
        new = ["g", "k", "p", "m"] if step == 0 else (["late"] if step == 3 else [])
        finished = {"k"} if step == 3 else set()
        active = [r for r in active if r not in finished] + new
        so = NS(scheduled_new_reqs=[NS(req_id=r, prompt_token_ids=prompts[r],
                                       sampling_params=params[r]) for r in new],
                finished_req_ids=finished, num_scheduled_tokens={r: 1 for r in active})
        assert runner.execute_model(so) is None
        mro = runner.sample_tokens(None)
        assert mro.req_ids == active
        assert [len(t) for t in mro.sampled_token_ids] == [1] * len(active)

        B = len(active)
        u = np.full((B, V), 0.5, np.float32)
        for i, r in enumerate(active):
            if r in mirror:
                u[i] = O.philox_uniforms(np.array([mirror[r].next_key()], np.int64), V)[0]
        sps = [params[r] for r in active]
        prm = O.make_params(B, [s.temperature for s in sps], [s.top_k for s in sps],
                            [s.top_p for s in sps], [s.min_p for s in sps],
                            [s.repetition_penalty for s in sps], [s.presence_penalty for s in sps],
                            [s.frequency_penalty for s in sps])
        pw = max(len(prompts[r]) for r in active)
        ow = max(1, max(len(outputs[r]) for r in active))
        pr = np.full((B, pw), V, np.int32)
        ou = np.full((B, ow), V, np.int32)
        for i, r in enumerate(active):
            pr[i, :len(prompts[r])] = prompts[r]
            ou[i, :len(outputs[r])] = outputs[r]
        L = 5 if any(params[r].logprobs for r in active) else None
        ref = O.sample(model.history[-1], prm, u, prompt_ids=pr, output_ids=ou, num_logprobs=L)
        got = [t[0] for t in mro.sampled_token_ids]
        assert got == ref["token"].tolist(), f"step {step}: {got} vs {ref['token'].tolist()}"
        if L is None:
            assert mro.logprobs is None
        else:
            assert mro.logprobs.logprob_token_ids == ref["lp_ids"].tolist()
            assert mro.logprobs.sampled_token_ranks == ref["ranks"].tolist()
            np.testing.assert_allclose(np.array(mro.logprobs.logprobs), ref["lp_vals"], rtol=1e-5,
                                       atol=1e-6)
        for r, tok in zip(active, got):
            outputs[r].append(tok)
    # the device history table agrees with the host lists, and so does the token-state table
    b = runner.input_batch
    assert (b.token_state is not None) == token_state
    for r in active:
        st = b.requests[r]
        n = len(outputs[r])
        assert b.output_ids[st.slot, :n].tolist() == outputs[r] and st.output_token_ids == outputs[r]
        assert int(b.output_lens[st.slot]) == n
        if token_state:
            want = np.zeros(V, np.uint32)
            np.add.at(want, np.array(outputs[r], np.int64), np.uint32(1))
            want[np.array(prompts[r], np.int64)] |= np.uint32(0x80000000)
            got = b.token_state[st.slot].cpu().numpy().view(np.uint32)
            assert np.array_equal(got, want), f"request {r}: token-state row differs"


def test_runner_logits_processors_match_oracle(cuda):
    from vllm_webgpu_amd.v1.sample.sampler import processor_lists

    V = 2048
    model = _FakeModel(V, cuda)
    runner = ROCmModelRunner(None, cuda, model, max_num_reqs=8, max_prompt_len=16,
                             max_output_len=16)
    params = {
        "bias": _sp(temperature=0.8, top_k=20, seed=31, logit_bias={7: 12.0, 8: -30.0}),
        "mint": _sp(temperature=0.0, min_tokens=3, stop_token_ids=[1, 2], eos_token_id=3),
        "bad": _sp(temperature=0.0, bad_words_token_ids=[[5], [1, 9]], repetition_penalty=1.2),
        "allow": _sp(temperature=1.0, seed=32, allowed_token_ids=[10, 11, 12, 13, 400]),
    }
    prompts = {"bias": [4], "mint": [1], "bad": [1], "allow": [10, 11]}
    mirror = {r: KeyStream(params[r].seed)
              for r in params if params[r].seed is not None}
    outputs = {r: [] for r in params}
    active = list(params)
    for step in range(4):
        so = NS(scheduled_new_reqs=[NS(req_id=r, prompt_token_ids=prompts[r],
                                       sampling_params=params[r]) for r in active] if step == 0 else [],
                finished_req_ids=set(), num_scheduled_tokens={r: 1 for r in active})
        runner.execute_model(so)
        md = runner.input_batch.make_sampling_metadata(active)
        mro = runner.sample_tokens(None)
        B = len(active)
        u = np.full((B, V), 0.5, np.float32)
        for i, r in enumerate(active):
            if r in mirror:
                u[i] = O.philox_uniforms(np.array([mirror[r].next_key()], np.int64), V)[0]
        sps = [params[r] for r in active]
        prm = O.make_params(B, [s.temperature for s in sps], [s.top_k for s in sps],
                            [s.top_p for s in sps], [s.min_p for s in sps],
                            [s.repetition_penalty for s in sps], [s.presence_penalty for s in sps],
                            [s.frequency_penalty for s in sps])
        pr = np.full((B, 2), V, np.int32)
        ou = np.full((B, max(1, step)), V, np.int32)
        for i, r in enumerate(active):
            pr[i, :len(prompts[r])] = prompts[r]
            ou[i, :len(outputs[r])] = outputs[r]
        ids, vals, _ = processor_lists(md, B, V)
        allowed = ~md.allowed_token_ids_mask.cpu().numpy()
        words = np.zeros((B, (V + 31) // 32 * 32), np.uint64)
        words[:, :V] = allowed
        bits = (words.reshape(B, -1, 32) << np.arange(32, dtype=np.uint64)).sum(axis=2).astype(np.uint32)
        ref = O.sample(model.history[-1], prm, u, prompt_ids=pr, output_ids=ou, allowed=bits,
                       adjust_ids=ids.numpy(), adjust_vals=vals.numpy())
        got = [t[0] for t in mro.sampled_token_ids]
        assert got == ref["token"].tolist(), f"step {step}: {got} vs {ref['token'].tolist()}"
        tok = dict(zip(active, got))
        assert tok["bad"] != 5 and tok["allow"] in (10, 11, 12, 13, 400)
        if step < 3:
            assert tok["mint"] not in (1, 2, 3)
        for r, t in zip(active, got):
            outputs[r].append(t)


def test_async_output_matches_sync(cuda):
    V = 1024
    outs = []
    for async_output in (False, True):
        model = _FakeModel(V, cuda)
        runner = ROCmModelRunner(None, cuda, model, max_num_reqs=4, max_prompt_len=8,
                                 max_output_len=8)
        params = {"a": _sp(temperature=0.7, top_k=10, seed=41, repetition_penalty=1.3),
                  "b": _sp(temperature=0.0, logprobs=3)}
        steps = []
        for step in range(3):
            so = NS(scheduled_new_reqs=[NS(req_id=r, prompt_token_ids=[1, 2], sampling_params=p)
                                        for r, p in params.items()] if step == 0 else [],
                    finished_req_ids=set(), num_scheduled_tokens={"a": 1, "b": 1})
            runner.execute_model(so)
            res = runner.sample_tokens(None, async_output=async_output)
            if async_output:
                assert hasattr(res, "get_output")
                res = res.get_output()
            steps.append((res.sampled_token_ids, res.logprobs.logprob_token_ids))
        outs.append(steps)
    assert outs[0] == outs[1]


def test_async_next_step_before_get_output(cuda):
    """execute_model of step N+1 runs before get_output() of step N: the model sees the same
    inputs and positions, and the steps sample the same tokens, as in the synchronous loop."""
    V = 1024
    runs = []
    for overlap in (False, True):
        model = _FakeModel(V, cuda)
        seen = []
        fwd = model.forward

        def forward(input_ids, positions, so, fwd=fwd, seen=seen):
            seen.append((input_ids.cpu().tolist(), positions.cpu().tolist()))
            return fwd(input_ids, positions, so)

        model.forward = forward
        runner = ROCmModelRunner(None, cuda, model, max_num_reqs=4, max_prompt_len=8,
                                 max_output_len=8)
        params = {"a": _sp(temperature=0.7, top_k=10, seed=41, repetition_penalty=1.3),
                  "b": _sp(temperature=0.0, presence_penalty=0.5, frequency_penalty=0.2)}
        pending, tokens = [], []
        for step in range(4):
            so = NS(scheduled_new_reqs=[NS(req_id=r, prompt_token_ids=[1, 2], sampling_params=p)
                                        for r, p in params.items()] if step == 0 else [],
                    finished_req_ids=set(), num_scheduled_tokens={"a": 1, "b": 1})
            runner.execute_model(so)
            if overlap and pending:
                tokens.append(pending.pop().get_output().sampled_token_ids)
            res = runner.sample_tokens(None, async_output=overlap)
            if overlap:
                pending.append(res)
            else:
                tokens.append(res.sampled_token_ids)
        if pending:
            tokens.append(pending.pop().get_output().sampled_token_ids)
        runs.append((tokens, seen))
    assert runs[0] == runs[1]
    # step 1's inputs are step 0's sampled ids, positions advance by one per step
    (tok, seen) = runs[0]
    assert seen[1][0] == [t[0] for t in tok[0]] and seen[1][1] == [2, 2]
    assert [p for _, p in seen] == [[1, 1], [2, 2], [3, 3], [4, 4]]


@pytest.mark.parametrize("logprobs", [None, 3])
def test_runner_structured_output_bitmask(cuda, logprobs):
    """sample_tokens(grammar_output): the structured-output rows sample inside their bitmask
    (without logprobs through the kernel's allowed mask; with logprobs the logits are masked
    first, so the raw logprobs see the mask, as in vLLM-v1), the other rows are untouched."""
    from vllm_webgpu_amd.v1.model_runner import grammar_words

    V = 3000
    model = _FakeModel(V, cuda)
    runner = ROCmModelRunner(None, cuda, model, max_num_reqs=4, max_prompt_len=8, max_output_len=8)
    params = {"free": _sp(temperature=0.9, top_k=40, seed=71, logprobs=logprobs),
              "json": _sp(temperature=0.9, top_p=0.9, seed=72, logprobs=logprobs),
              "g": _sp(temperature=0.0, logprobs=logprobs)}
    rng = np.random.default_rng(73)
    mirror = {r: KeyStream(params[r].seed)
              for r in params if params[r].seed is not None}
    active = list(params)
    so = NS(scheduled_new_reqs=[NS(req_id=r, prompt_token_ids=[1, 2], sampling_params=params[r])
                                for r in active], finished_req_ids=set(),
            num_scheduled_tokens={r: 1 for r in active})
    runner.execute_model(so)
    W = (V + 31) // 32
    bm = np.zeros((2, W), np.int64)
    for i in range(2):
        for t in rng.choice(V, 25, replace=False):
            bm[i, t >> 5] |= 1 << (t & 31)
    bm = (bm - (bm >= 2 ** 31) * 2 ** 32).astype(np.int32)
    go = NS(structured_output_request_ids=["json", "g"], grammar_bitmask=bm)
    mro = runner.sample_tokens(go)
    words = grammar_words(go, active, V, torch.device("cpu")).numpy().view(np.uint32)
    B = len(active)
    u = np.full((B, V), 0.5, np.float32)
    for i, r in enumerate(active):
        if r in mirror:
            u[i] = O.philox_uniforms(np.array([mirror[r].next_key()], np.int64), V)[0]
    sps = [params[r] for r in active]
    prm = O.make_params(B, [s.temperature for s in sps], [s.top_k for s in sps],
                        [s.top_p for s in sps], [s.min_p for s in sps],
                        [s.repetition_penalty for s in sps], [s.presence_penalty for s in sps],
                        [s.frequency_penalty for s in sps])
    x = model.history[-1].copy()
    allowed_bits = ((words[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(B, -1)[:, :V]
    if logprobs is None:
        ref = O.sample(x, prm, u, allowed=words)
    else:
        x[allowed_bits == 0] = -np.inf
        ref = O.sample(x, prm, u, num_logprobs=logprobs)
    got = [t[0] for t in mro.sampled_token_ids]
    assert got == ref["token"].tolist()
    for i in (1, 2):
        assert allowed_bits[i, got[i]] == 1
    if logprobs is not None:
        assert mro.logprobs.logprob_token_ids == ref["lp_ids"].tolist()
        np.testing.assert_allclose(np.array(mro.logprobs.logprobs), ref["lp_vals"], rtol=1e-5, atol=1e-6)
