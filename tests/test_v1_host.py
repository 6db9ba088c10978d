"""Host logic of the vLLM-v1 front end (no GPU): metadata packing from the persistent batch,
device-side history appends (exercised on CPU tensors), uniform draws, padding, and the loud
failures the sampler owes its callers (no CPU fallback, unsupported processors refused)."""
from types import SimpleNamespace as NS

import numpy as np
import pytest
import torch

from vllm_webgpu_amd.v1.model_runner import InputBatch, ROCmModelRunner, WebGPUModelRunner
from vllm_webgpu_amd.v1.outputs import LogprobsTensors, ModelRunnerOutput, SamplerOutput
from vllm_webgpu_amd.v1.sample.metadata import SamplingMetadata
from vllm_webgpu_amd.v1.sample.sampler import (Sampler, draw_seeds, pad_output_ids,
                                                processor_lists)

V = 100


def sp(**kw):
    base = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0,
                presence_penalty=0.0, frequency_penalty=0.0, seed=None, logprobs=None)
    base.update(kw)
    return NS(**base)


def test_pad_output_ids_ragged():
    ids, lens = pad_output_ids([[1, 2, 3], [], [7]], V, torch.device("cpu"))
    assert ids.dtype == torch.int32 and ids.tolist() == [[1, 2, 3], [V, V, V], [7, V, V]]
    assert lens.tolist() == [3, 0, 1]
    ids, lens = pad_output_ids([[], []], V, torch.device("cpu"))
    assert ids.shape == (2, 1) and ids.eq(V).all() and lens.tolist() == [0, 0]


def test_draw_seeds_seeded_rows_reproducible():
    g1 = torch.Generator().manual_seed(5)
    s1 = draw_seeds(3, {1: g1}, torch.device("cpu"))
    assert s1.dtype == torch.int64 and s1.shape == (3,)
    g2 = torch.Generator().manual_seed(5)
    s2 = draw_seeds(3, {1: g2}, torch.device("cpu"))
    assert s1[1] == s2[1]                     # seeded row reproducible
    assert s1[0] != s2[0] or s1[2] != s2[2]   # unseeded rows are fresh draws
    assert draw_seeds(3, {1: g2}, torch.device("cpu"))[1] != s1[1]  # next step: a new key


def test_input_batch_metadata_fields():
    b = InputBatch(4, 8, 6, V, torch.device("cpu"))
    b.add_request("a", [1, 2, 3], sp(temperature=0.0))
    b.add_request("b", [4, 5], sp(temperature=0.7, top_k=20, top_p=0.9, seed=11, logprobs=3,
                                  repetition_penalty=1.2))
    b.add_request("c", [6], sp(temperature=1.0, top_k=-1, min_p=0.05, logprobs=1))
    m = b.make_sampling_metadata(["c", "a", "b"])
    assert isinstance(m, SamplingMetadata)
    assert not m.all_greedy and not m.all_random
    assert m.temperature.tolist() == pytest.approx([1.0, 0.0, 0.7])
    assert m.top_k.tolist() == [0, 0, 20]           # -1 normalised to "off"
    assert m.top_p.tolist() == pytest.approx([1.0, 1.0, 0.9])
    assert m.min_p.tolist() == pytest.approx([0.05, 0.0, 0.0])
    assert m.max_num_logprobs == 3
    assert set(m.generators) == {2}                 # only the seeded random row
    assert not m.no_penalties
    assert m.prompt_token_ids.tolist()[1] == [1, 2, 3]   # widest prompt: 3 columns
    assert m.prompt_token_ids.tolist()[0] == [6, V, V]
    assert m.output_token_ids_tensor.eq(V).all() and m.output_token_lens.tolist() == [0, 0, 0]


def test_input_batch_all_greedy_and_off_switches():
    b = InputBatch(2, 4, 4, V, torch.device("cpu"))
    b.add_request("a", [1], sp(temperature=0.0))
    b.add_request("b", [2], sp(temperature=1e-6))
    m = b.make_sampling_metadata(["a", "b"])
    assert m.all_greedy and m.temperature is None
    assert m.top_k is None and m.top_p is None and m.min_p is None
    assert m.no_penalties and m.prompt_token_ids is None and m.output_token_ids_tensor is None
    assert m.max_num_logprobs is None


def test_input_batch_append_and_slot_reuse():
    b = InputBatch(2, 4, 3, V, torch.device("cpu"))
    b.add_request("a", [1], sp(repetition_penalty=1.1))
    b.add_request("b", [2], sp(repetition_penalty=1.1))
    with pytest.raises(RuntimeError):
        b.add_request("c", [3], sp())
    for step in range(4):   # the table holds 3 ids: the 4th append is dropped, not wrapped
        b.append_sampled(["b", "a"], torch.tensor([10 + step, 20 + step], dtype=torch.int32))
    sa, sb = b.requests["a"].slot, b.requests["b"].slot
    assert b.output_ids[sa].tolist() == [20, 21, 22] and b.output_ids[sb].tolist() == [10, 11, 12]
    assert b.output_lens[sa].item() == 3
    b.remove_request("a")
    b.add_request("c", [9, 9], sp())
    assert b.requests["c"].slot == sa
    assert b.output_ids[sa].eq(V).all() and b.output_lens[sa].item() == 0
    assert b.prompt_ids[sa].tolist()[:3] == [9, 9, V]
    with pytest.raises(ValueError):
        b.add_request("d", [1] * 5, sp())          # longer than max_prompt_len
    with pytest.raises(ValueError):
        b.add_request("c", [1], sp())              # duplicate id


def test_input_batch_decode_inputs_from_device_tables():
    """The next step's inputs come from the device tables and the sampled-step count, not from
    the host lists (which lag while a step's output is in flight)."""
    b = InputBatch(3, 4, 2, V, torch.device("cpu"))
    b.add_request("a", [5, 6, 7], sp())
    b.add_request("b", [9], sp())
    b.add_request("e", [], sp())
    ids, pos = b.decode_inputs(["a", "b", "e"])
    assert ids.dtype == torch.int32 and ids.tolist() == [7, 9, 0] and pos.tolist() == [2, 0, -1]
    b.append_sampled(["b", "a"], torch.tensor([40, 41], dtype=torch.int32))
    assert b.requests["a"].output_token_ids == [] and b.requests["a"].num_sampled == 1
    ids, pos = b.decode_inputs(["a", "b"])
    assert ids.tolist() == [41, 40] and pos.tolist() == [3, 1]
    b.append_sampled(["a"], torch.tensor([42], dtype=torch.int32))
    assert b.decode_inputs(["a"])[0].tolist() == [42]
    b.append_sampled(["a"], torch.tensor([43], dtype=torch.int32))   # past max_output_len
    with pytest.raises(ValueError):
        b.decode_inputs(["a"])


def test_sampler_refuses_cpu_logits_and_unsupported_modes():
    s = Sampler()
    b = InputBatch(1, 2, 2, V, torch.device("cpu"))
    b.add_request("a", [1], sp())
    m = b.make_sampling_metadata(["a"])
    with pytest.raises(ValueError, match="ROCm device"):
        s(torch.zeros(1, V), m)                    # no host fallback
    with pytest.raises(NotImplementedError):
        Sampler(logprobs_mode="processed_logprobs")
    for bad in (0.0, -1.0, float("nan"), float("inf")):
        with pytest.raises(ValueError, match="logit_softcap"):
            Sampler(logit_softcap=bad)
    assert Sampler(logit_softcap=30.0).logit_softcap == 30.0
    assert WebGPUModelRunner(None, device="cpu", logit_softcap=30.0).sampler.logit_softcap == 30.0


def _meta(**kw):
    base = dict(temperature=None, all_greedy=True, all_random=False, top_p=None, top_k=None,
                generators={}, max_num_logprobs=None, no_penalties=True, prompt_token_ids=None,
                frequency_penalties=None, presence_penalties=None, repetition_penalties=None,
                output_token_ids=[[], []])
    base.update(kw)
    return SamplingMetadata(**base)


def test_processor_lists_bad_words_min_tokens_and_bias():
    m = _meta(output_token_ids=[[5, 6, 7], [9]],
              bad_words_token_ids={0: [[3], [6, 7, 11], [5, 12], [1, 2, 3, 4, 5, 13]],
                                   1: [[9, 14], [8, 15]]},
              min_tokens={0: (2, {0}), 1: (3, {0, 2})},
              logit_bias=[None, {4: 1.5, 20: -2.0}])
    ids, vals, lens = processor_lists(m, 2, V)
    rows = [{(int(t), float(v)) for t, v in zip(ids[i].tolist(), vals[i].tolist()) if t < V}
            for i in range(2)]
    ninf = float("-inf")
    # row 0: [3] always, [6, 7, 11] matches the output tail, [5, 12] does not, too long skipped;
    # min_tokens 2 already reached
    assert rows[0] == {(3, ninf), (11, ninf)}
    # row 1: [9, 14] matches, [8, 15] does not; min_tokens 3 not reached -> stop ids 0, 2; bias
    assert rows[1] == {(14, ninf), (0, ninf), (2, ninf), (4, 1.5), (20, -2.0)}
    assert ids.shape[1] == 5 and (ids[0, 2:] == V).all()          # padded with V
    assert lens.tolist() == [2, 5]
    assert processor_lists(_meta(), 2, V) is None


def test_pack_allowed_bits():
    from vllm_webgpu_amd.ops import pack_allowed
    allowed = torch.zeros(2, 70, dtype=torch.bool)
    allowed[0, [0, 31, 32, 69]] = True
    allowed[1] = True
    w = pack_allowed(allowed)
    assert w.dtype == torch.int32 and w.shape == (2, 3)
    u = w.to(torch.int64) & 0xFFFFFFFF
    assert u[0].tolist() == [1 | (1 << 31), 1, 1 << 5]
    assert u[1].tolist() == [0xFFFFFFFF, 0xFFFFFFFF, (1 << 6) - 1]


def test_input_batch_processor_fields():
    b = InputBatch(2, 4, 4, V, torch.device("cpu"))
    b.add_request("a", [1], NS(temperature=0.0, logit_bias={3: 2.0}, min_tokens=2,
                                stop_token_ids=[7], eos_token_id=0,
                                bad_words_token_ids=[[5]], allowed_token_ids=None))
    b.add_request("b", [2], NS(temperature=1.0, allowed_token_ids=[1, 2, 3]))
    m = b.make_sampling_metadata(["a", "b"])
    assert m.logit_bias == [{3: 2.0}, None]
    assert m.min_tokens == {0: (2, {0, 7})}
    assert m.bad_words_token_ids == {0: [[5]]}
    assert m.allowed_token_ids_mask.shape == (2, V)
    assert not m.allowed_token_ids_mask[0].any()
    assert m.allowed_token_ids_mask[1].sum() == V - 3 and not m.allowed_token_ids_mask[1, 1:4].any()


def test_min_tokens_and_bad_words_with_an_output_in_flight():
    """While a step's output is in flight (async output) the host copy of a request's output
    lags the device by a token: min-tokens is decided on the device-side count, and bad words
    (which match the host copy) refuse to sample until get_output() has caught it up."""
    b = InputBatch(2, 4, 8, V, torch.device("cpu"))
    b.add_request("a", [1], NS(temperature=1.0, min_tokens=2, stop_token_ids=[7], eos_token_id=0))
    b.add_request("w", [2], NS(temperature=1.0, bad_words_token_ids=[[5, 6]]))
    st = b.requests["a"]
    st.output_token_ids, st.num_sampled = [4], 2     # second sampled id not on the host yet
    m = b.make_sampling_metadata(["a"])
    assert m.min_tokens == {}                        # the minimum is reached on the device
    st.num_sampled = 1
    st.output_token_ids = []
    assert b.make_sampling_metadata(["a"]).min_tokens == {0: (2, {0, 7})}
    b.requests["w"].num_sampled = 1                  # its host list is still empty
    with pytest.raises(RuntimeError, match="get_output"):
        b.make_sampling_metadata(["a", "w"])
    b.requests["w"].output_token_ids = [5]
    assert b.make_sampling_metadata(["a", "w"]).bad_words_token_ids == {1: [[5, 6]]}


def test_runner_without_model_and_grammar():
    r = WebGPUModelRunner(None, device="cpu")
    assert r is not None and WebGPUModelRunner is ROCmModelRunner
    assert r.execute_model(NS()) is None and r.sample_tokens(None) is None
    with pytest.raises(NotImplementedError):
        r.load_model()
    assert r.supported_worker_tasks() == ("generate",)


def test_output_containers():
    lp = LogprobsTensors(torch.tensor([[3, 1, 2]], dtype=torch.int32),
                         torch.tensor([[-1.5, -0.5, -1.0]]), torch.tensor([3], dtype=torch.int32))
    lists = lp.tolists()
    assert lists.logprob_token_ids == [[3, 1, 2]] and lists.sampled_token_ranks == [3]
    out = SamplerOutput(sampled_token_ids=torch.tensor([[3]], dtype=torch.int32), logprobs_tensors=lp)
    assert out.sampled_token_ids.shape == (1, 1)
    mro = ModelRunnerOutput(req_ids=["x"], req_id_to_index={"x": 0}, sampled_token_ids=[[3]],
                            logprobs=lists)
    assert mro.req_id_to_index["x"] == 0


def test_platform_routes_to_worker():
    from vllm_webgpu_amd.platform import WORKER_CLS, MI355XPlatform, WebGPUPlatform
    cfg = NS(parallel_config=NS(worker_cls="auto", distributed_executor_backend=None))
    WebGPUPlatform.check_and_update_config(cfg)
    assert cfg.parallel_config.worker_cls == WORKER_CLS
    assert cfg.parallel_config.distributed_executor_backend == "uni"
    mod, cls = WORKER_CLS.rsplit(".", 1)
    import importlib
    assert getattr(importlib.import_module(mod), cls) is not None
    assert MI355XPlatform.is_pin_memory_available()


def test_grammar_words_and_in_place_mask():
    """vLLM-v1 GrammarOutput -> per-row allowed words in request order (rows without a grammar
    allow everything), and the in-place -inf mask used when logprobs are requested."""
    from vllm_webgpu_amd.v1.model_runner import apply_grammar_words, grammar_words
    Vg = 70
    bm = np.zeros((2, 3), np.int32)
    bm[0] = [0b101, 0, 1 << 5]          # tokens 0, 2 and 69
    bm[1, 0] = -1                       # tokens 0..31
    go = NS(structured_output_request_ids=["b", "c"], grammar_bitmask=bm)
    w = grammar_words(go, ["a", "b", "c"], Vg, torch.device("cpu"))
    assert w[0].tolist() == [-1, -1, -1] and w[1].tolist() == bm[0].tolist()
    assert grammar_words(NS(structured_output_request_ids={"c": 0}, grammar_bitmask=bm), ["c"], Vg,
                         torch.device("cpu"))[0].tolist() == bm[0].tolist()
    assert grammar_words(None, ["a"], Vg, torch.device("cpu")) is None
    x = torch.zeros(3, Vg)
    apply_grammar_words(x, w)
    assert torch.isfinite(x[0]).all()
    assert torch.isfinite(x[1]).nonzero().flatten().tolist() == [0, 2, 69]
    assert torch.isfinite(x[2]).nonzero().flatten().tolist() == list(range(32))
    with pytest.raises(ValueError):
        grammar_words(NS(structured_output_request_ids=["a"], grammar_bitmask=bm[:, :2]), ["a"], Vg,
                      torch.device("cpu"))


def test_sampler_config_from_env(monkeypatch):
    """The VLLM_WEBGPU_AMD_* variables in the reference's envs/config pattern: defaults,
    parsing and validation that names the variable."""
    from vllm_webgpu_amd import config, envs
    for k in list(envs.environment_variables):
        monkeypatch.delenv(k, raising=False)
    config.reset_config()
    c = config.get_config()
    assert (c.token_state, c.async_output, c.coop_wait_polls, c.max_num_reqs, c.debug) == \
        (True, False, 1 << 20, 1024, False)
    monkeypatch.setenv("VLLM_WEBGPU_AMD_TOKEN_STATE", "0")
    monkeypatch.setenv("VLLM_WEBGPU_AMD_ASYNC_OUTPUT", "true")
    monkeypatch.setenv("VLLM_WEBGPU_AMD_MAX_NUM_REQS", "64")
    config.reset_config()
    c = config.get_config()
    assert (c.token_state, c.async_output, c.max_num_reqs) == (False, True, 64)
    monkeypatch.setenv("VLLM_WEBGPU_AMD_COOP_WAIT_POLLS", "-3")
    with pytest.raises(ValueError, match="VLLM_WEBGPU_AMD_COOP_WAIT_POLLS"):
        config.SamplerConfig.from_env()
    monkeypatch.setenv("VLLM_WEBGPU_AMD_COOP_WAIT_POLLS", "x")
    with pytest.raises(ValueError, match="sampler environment"):
        config.SamplerConfig.from_env()
    with pytest.raises(AttributeError):
        envs.VLLM_WEBGPU_AMD_NOPE
    config.reset_config()


def test_key_stream_splitmix64():
    """Seeded requests' per-step keys: SplitMix64 (Steele, Lea, Flood 2014) of the seed advanced
    by the golden-ratio increment -- the first outputs for seed 0 are the published
    0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f -- and draw_seeds advances
    each stream by one key per step, computing a batch's keys together."""
    from vllm_webgpu_amd.v1.sample.sampler import KeyStream
    k = KeyStream(0)
    got = [k.next_key() & 0xFFFFFFFFFFFFFFFF for _ in range(3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    a, b = KeyStream(1234), KeyStream(1234)
    s = draw_seeds(4, {1: a, 3: KeyStream(99)}, torch.device("cpu"))
    assert int(s[1]) == b.next_key() and a.step == 1
    s2 = draw_seeds(4, {1: a}, torch.device("cpu"))
    assert int(s2[1]) == b.next_key() and int(s2[1]) != int(s[1])
