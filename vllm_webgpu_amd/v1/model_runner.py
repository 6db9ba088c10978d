"""Model runner: caches device logits in ``execute_model`` and samples them in ``sample_tokens``.

Mirrors the sampling half of ``WebGPUModelRunner`` (``vllm_webgpu/v1/model_runner.py:54-176``):
same method names (``execute_model``, ``sample_tokens``, ``supported_worker_tasks``,
``reset_mm_cache``, ``reset_encoder_cache``), same ``_last_logits`` cache (``:63,140``), same
decode-only batching rule (``:129-137``: the last token of each request, position = length - 1).
Where the reference argmaxes numpy logits on the host and returns ``None`` from
``sample_tokens`` (``:145,164-166``), this runner keeps the logits on the GPU, builds a vLLM-v1
``SamplingMetadata`` from a persistent batch and calls the device ``Sampler``.

The persistent batch (``InputBatch``) holds every running request's prompt and generated ids in
device tables padded with ``vocab_size``; each step gathers the scheduled rows and, after
sampling, appends the sampled ids on the device, so histories are never re-uploaded.  On a GPU
it also keeps a token-state table, one uint32 word per (request slot, token): prompt flag and
output count, set when a request is admitted and counted once per sampled id
(``vws_token_state_update``), with a bitmap of its non-zero words.  The penalties read that
table at the tokens that reach the sampler's candidates, and the bitmap lets rows that top-p
alone cuts buffer their history tokens, so a long prompt or output costs nothing per step
(vLLM-v1 rebuilds the same prompt mask and output bin counts from the histories every step).  Host
copies of the generated ids (needed by ``SamplingMetadata.output_token_ids`` and the engine)
come from the one device-to-host copy of the sampled ids per step.

Building the model and its weights is outside this package: ``model`` is any object with the
reference model's ``forward(input_ids, positions, scheduler_output) -> logits [B, V]``
(``vllm_webgpu/models/llama.py:222-237``) that returns a ROCm-device tensor.
"""
from __future__ import annotations

import logging
from dataclasses import dataclass, field
from typing import Any

import torch

from .outputs import ModelRunnerOutput
from .sample.metadata import SamplingMetadata
from .sample.sampler import KeyStream, Sampler

logger = logging.getLogger(__name__)

_SAMPLING_EPS = 1e-5


def _param(sp: Any, name: str, default):
    v = getattr(sp, name, default) if sp is not None else default
    return default if v is None else v


@dataclass
class CachedRequestState:
    req_id: str
    prompt_token_ids: list[int]
    sampling_params: Any
    generator: KeyStream | None
    slot: int
    output_token_ids: list[int] = field(default_factory=list)
    # ids sampled on the device so far; counted when the step samples, so it leads the host
    # list above while a step's output is still in flight (async output)
    num_sampled: int = 0

    @property
    def num_tokens(self) -> int:
        return len(self.prompt_token_ids) + self.num_sampled


class InputBatch:
    """Persistent per-request sampling state, resident on the device between steps.

    Slots are reused as requests finish.  ``prompt_ids[slot]`` / ``output_ids[slot]`` hold the
    request's ids padded with ``vocab_size`` (the padding id the sampler ignores);
    ``output_lens[slot]`` counts the generated ids.
    """

    def __init__(self, max_num_reqs: int, max_prompt_len: int, max_output_len: int,
                 vocab_size: int, device: torch.device, token_state: bool = True) -> None:
        self.max_num_reqs = max_num_reqs
        self.max_prompt_len = max_prompt_len
        self.max_output_len = max_output_len
        self.vocab_size = vocab_size
        self.device = device
        self.prompt_ids = torch.full((max_num_reqs, max(max_prompt_len, 1)), vocab_size,
                                     dtype=torch.int32, device=device)
        self.output_ids = torch.full((max_num_reqs, max(max_output_len, 1)), vocab_size,
                                     dtype=torch.int32, device=device)
        self.output_lens = torch.zeros(max_num_reqs, dtype=torch.int32, device=device)
        # per-slot token state (prompt flag | output count), on a ROCm device only: the table
        # is maintained by the library's kernels
        self.token_state = self.token_state_bits = None
        if token_state and torch.device(device).type == "cuda":
            self.token_state_bits = torch.zeros((max_num_reqs, (vocab_size + 31) // 32),
                                                dtype=torch.int32, device=device)
            self.token_state = torch.zeros((max_num_reqs, vocab_size), dtype=torch.int32,
                                           device=device)
        self.requests: dict[str, CachedRequestState] = {}
        self._free = list(range(max_num_reqs - 1, -1, -1))

    def add_request(self, req_id: str, prompt_token_ids: list[int], sampling_params: Any) -> int:
        if req_id in self.requests:
            raise ValueError(f"request {req_id!r} is already in the batch")
        if len(prompt_token_ids) > self.max_prompt_len:
            raise ValueError(f"prompt of {len(prompt_token_ids)} tokens exceeds "
                             f"max_prompt_len={self.max_prompt_len}")
        if not self._free:
            raise RuntimeError(f"batch is full ({self.max_num_reqs} requests)")
        slot = self._free.pop()
        seed = _param(sampling_params, "seed", None)
        gen = KeyStream(int(seed)) if seed is not None else None
        self.requests[req_id] = CachedRequestState(req_id, list(prompt_token_ids),
                                                   sampling_params, gen, slot)
        row = torch.full((self.prompt_ids.shape[1],), self.vocab_size, dtype=torch.int32)
        if prompt_token_ids:
            row[:len(prompt_token_ids)] = torch.as_tensor(prompt_token_ids, dtype=torch.int32)
        self.prompt_ids[slot].copy_(row, non_blocking=False)
        self.output_ids[slot].fill_(self.vocab_size)
        self.output_lens[slot] = 0
        if self.token_state is not None:
            from .. import ops

            self.token_state[slot].zero_()
            self.token_state_bits[slot].zero_()
            if prompt_token_ids:
                ops.token_state_update(self.token_state, self.prompt_ids[slot, :len(prompt_token_ids)],
                                       rows=slot, prompt=True, bits=self.token_state_bits)
        return slot

    def remove_request(self, req_id: str) -> None:
        st = self.requests.pop(req_id, None)
        if st is not None:
            self._free.append(st.slot)

    def make_sampling_metadata(self, req_ids: list[str]) -> SamplingMetadata:
        states = [self.requests[r] for r in req_ids]
        dev = self.device
        B = len(states)
        sps = [s.sampling_params for s in states]
        temp = [float(_param(sp, "temperature", 1.0)) for sp in sps]
        greedy = [t < _SAMPLING_EPS for t in temp]
        top_k = [int(_param(sp, "top_k", 0)) for sp in sps]
        top_k = [0 if k < 0 else k for k in top_k]            # -1 and 0 both mean "off"
        top_p = [float(_param(sp, "top_p", 1.0)) for sp in sps]
        min_p = [float(_param(sp, "min_p", 0.0)) for sp in sps]
        rep = [float(_param(sp, "repetition_penalty", 1.0)) for sp in sps]
        pres = [float(_param(sp, "presence_penalty", 0.0)) for sp in sps]
        freq = [float(_param(sp, "frequency_penalty", 0.0)) for sp in sps]
        lps = [_param(sp, "logprobs", None) for sp in sps]
        lps = [int(x) for x in lps if x is not None]
        # logits processors (vLLM-v1 SamplingParams fields)
        bias = [_param(sp, "logit_bias", None) for sp in sps]
        bad = {i: [list(w) for w in _param(sp, "bad_words_token_ids", [])]
               for i, sp in enumerate(sps) if _param(sp, "bad_words_token_ids", None)}
        # bad words match the end of the host copy of the output, which lags the device while a
        # step's output is in flight (async output): refuse rather than match stale ids
        stale = [states[i].req_id for i in bad
                 if states[i].num_sampled != len(states[i].output_token_ids)]
        if stale:
            raise RuntimeError(f"requests {stale} use bad words while a step's output is still in "
                               "flight: call get_output() on it before sampling the next step")
        mint = {}
        for i, sp in enumerate(sps):
            mt = int(_param(sp, "min_tokens", 0))
            # counted on the device side (num_sampled), which is current even while the host
            # copy of the output lags (async output); rows past the minimum are left out
            if mt > 0 and states[i].num_sampled < mt:
                stop = set(_param(sp, "stop_token_ids", [])) | set(_param(sp, "all_stop_token_ids", []))
                eos = _param(sp, "eos_token_id", None)
                if eos is not None:
                    stop.add(int(eos))
                mint[i] = (mt, stop)
        allowed_rows = [_param(sp, "allowed_token_ids", None) for sp in sps]
        allowed_mask = None
        if any(a is not None for a in allowed_rows):
            allowed_mask = torch.zeros((B, self.vocab_size), dtype=torch.bool)
            for i, ids in enumerate(allowed_rows):
                if ids is not None:
                    allowed_mask[i] = True
                    allowed_mask[i, torch.as_tensor(list(ids), dtype=torch.int64)] = False
            allowed_mask = allowed_mask.to(dev, non_blocking=True)

        def t(x, dtype):
            return torch.tensor(x, dtype=dtype).to(dev, non_blocking=True)

        all_greedy = all(greedy)
        no_penalties = all(r == 1.0 for r in rep) and not any(pres) and not any(freq)
        slots = t([s.slot for s in states], torch.int64)
        table = self.token_state is not None and not no_penalties
        # gather only the populated columns: the kernel reads every history column it is given
        pw = max(1, max((len(s.prompt_token_ids) for s in states), default=1))
        ow = max(1, min(self.output_ids.shape[1],
                        max((s.num_sampled for s in states), default=1)))
        # Rows that are not random draw uniforms too (one [B, V] draw), but the kernel ignores them.
        gens = {i: s.generator for i, s in enumerate(states)
                if s.generator is not None and not greedy[i]}
        return SamplingMetadata(
            temperature=None if all_greedy else t(temp, torch.float32),
            all_greedy=all_greedy,
            all_random=not any(greedy),
            top_p=None if all(p >= 1.0 for p in top_p) else t(top_p, torch.float32),
            top_k=None if not any(top_k) else t(top_k, torch.int32),
            generators=gens,
            max_num_logprobs=max(lps) if lps else None,
            no_penalties=no_penalties,
            prompt_token_ids=(None if no_penalties or table
                              else self.prompt_ids[:, :pw].index_select(0, slots)),
            frequency_penalties=t(freq, torch.float32),
            presence_penalties=t(pres, torch.float32),
            repetition_penalties=t(rep, torch.float32),
            output_token_ids=[s.output_token_ids for s in states],
            min_p=None if not any(min_p) else t(min_p, torch.float32),
            allowed_token_ids_mask=allowed_mask,
            bad_words_token_ids=bad,
            min_tokens=mint,
            logit_bias=bias if any(bias) else None,
            output_token_ids_tensor=(None if no_penalties or table
                                    else self.output_ids[:, :ow].index_select(0, slots)),
            output_token_lens=(None if no_penalties or table
                               else self.output_lens.index_select(0, slots)),
            token_state=self.token_state if table else None,
            token_state_rows=slots.to(torch.int32) if table else None,
            token_state_bits=self.token_state_bits if table else None,
        ) if B else None

    def decode_inputs(self, req_ids: list[str]) -> tuple[torch.Tensor, torch.Tensor]:
        """The next decode step's inputs, int32 [B] on the device: each request's last token
        (its newest sampled id, read from the device table, else the last prompt id) and its
        position (number of tokens - 1).  Nothing waits for a step's output to reach the host,
        so the next step can be scheduled while the previous one's ids are still in flight."""
        states = [self.requests[r] for r in req_ids]
        over = [s.req_id for s in states if s.num_sampled > self.output_ids.shape[1]]
        if over:
            raise ValueError(f"requests {over} generated more than max_output_len="
                             f"{self.output_ids.shape[1]} tokens")
        dev = self.device
        slots = torch.tensor([s.slot for s in states], dtype=torch.int64, device=dev)
        ocol = torch.tensor([max(s.num_sampled - 1, 0) for s in states], dtype=torch.int64,
                            device=dev)
        pcol = torch.tensor([max(len(s.prompt_token_ids) - 1, 0) for s in states],
                            dtype=torch.int64, device=dev)
        has_out = torch.tensor([s.num_sampled > 0 for s in states], device=dev)
        has_prompt = torch.tensor([len(s.prompt_token_ids) > 0 for s in states], device=dev)
        last_out = self.output_ids[slots, ocol]
        last_prompt = self.prompt_ids[slots, pcol]
        zero = torch.zeros_like(last_out)
        input_ids = torch.where(has_out, last_out, torch.where(has_prompt, last_prompt, zero))
        positions = torch.tensor([s.num_tokens - 1 for s in states], dtype=torch.int32, device=dev)
        return input_ids, positions

    def append_sampled(self, req_ids: list[str], sampled: torch.Tensor) -> None:
        """Appends ``sampled`` (int32 [B] on the device) to the output tables, on the device,
        and counts the step in each request's ``num_sampled``."""
        if not req_ids:
            return
        for r in req_ids:
            self.requests[r].num_sampled += 1
        slots = torch.tensor([self.requests[r].slot for r in req_ids], dtype=torch.int64,
                             device=self.device)
        pos = self.output_lens.index_select(0, slots).long()
        ok = pos < self.output_ids.shape[1]
        self.output_ids[slots[ok], pos[ok]] = sampled.to(torch.int32)[ok]
        self.output_lens.index_add_(0, slots, ok.to(torch.int32))
        if self.token_state is not None:
            from .. import ops

            ops.token_state_update(self.token_state, sampled, rows=slots.to(torch.int32),
                                   bits=self.token_state_bits)


def grammar_words(grammar_output: Any, req_ids: list[str], vocab_size: int,
                  device: torch.device) -> torch.Tensor | None:
    """int32 [B, ceil(V/32)] allowed-token words of a step's structured-output rows, rows in
    ``req_ids`` order (bit t & 31 of word t >> 5 set = token t allowed; rows without a grammar
    allow everything), from vLLM-v1's ``GrammarOutput``: ``grammar_bitmask`` int32
    [n, ceil(V/32)] and ``structured_output_request_ids`` (a list of request ids, or a dict of
    request id -> bitmask row).  None when the step has no bitmask."""
    bm = getattr(grammar_output, "grammar_bitmask", None) if grammar_output is not None else None
    if bm is None:
        return None
    ids = getattr(grammar_output, "structured_output_request_ids", None) or []
    row_of = dict(ids) if isinstance(ids, dict) else {r: i for i, r in enumerate(ids)}
    bm = torch.as_tensor(bm, dtype=torch.int32)
    W = (vocab_size + 31) // 32
    if bm.dim() != 2 or bm.shape[1] < W:
        raise ValueError(f"grammar_bitmask must be [n, >= {W}] int32 words (got {tuple(bm.shape)})")
    words = torch.full((len(req_ids), W), -1, dtype=torch.int32)
    for i, r in enumerate(req_ids):
        j = row_of.get(r)
        if j is not None:
            words[i] = bm[j, :W]
    return words.to(device, non_blocking=True)


def apply_grammar_words(logits: torch.Tensor, words: torch.Tensor) -> torch.Tensor:
    """Sets the logits of tokens outside ``words`` to -inf, in place (vLLM-v1 applies the
    grammar bitmask to the logits before its sampler, so raw logprobs see the mask)."""
    B, V = logits.shape
    shifts = torch.arange(32, dtype=torch.int32, device=logits.device)
    bits = (words.unsqueeze(-1) >> shifts) & 1
    allowed = bits.reshape(B, -1)[:, :V].bool()
    return logits.masked_fill_(~allowed, float("-inf"))


class AsyncModelRunnerOutput:
    """A step's output whose device-to-host copy is in flight (vLLM-v1's async output)."""

    def __init__(self, batch: InputBatch, req_ids: list[str], sampled: torch.Tensor,
                 logprobs: Any) -> None:
        pin = sampled.is_cuda
        self._batch, self._req_ids = batch, req_ids
        self._ids = torch.empty(sampled.shape, dtype=sampled.dtype, pin_memory=pin)
        self._ids.copy_(sampled, non_blocking=pin)
        self._lp = None
        if logprobs is not None:
            self._lp = tuple(torch.empty(t.shape, dtype=t.dtype, pin_memory=pin) for t in logprobs)
            for h, d in zip(self._lp, logprobs):
                h.copy_(d, non_blocking=pin)
        self._event = None
        if pin:
            self._event = torch.cuda.Event()
            self._event.record()
        self._result: ModelRunnerOutput | None = None

    def get_output(self) -> ModelRunnerOutput:
        if self._result is None:
            if self._event is not None:
                self._event.synchronize()
            ids = self._ids.tolist()
            for r, tok in zip(self._req_ids, ids):
                self._batch.requests[r].output_token_ids.append(tok)
            lp = None
            if self._lp is not None:
                from .outputs import LogprobsTensors
                lp = LogprobsTensors(*self._lp).tolists()
            req_ids = self._req_ids
            self._result = ModelRunnerOutput(
                req_ids=list(req_ids), req_id_to_index={r: i for i, r in enumerate(req_ids)},
                sampled_token_ids=[[t] for t in ids], logprobs=lp, prompt_logprobs_dict={},
                pooler_output=[])
        return self._result


class ROCmModelRunner:
    """Runner for one MI355X: model forward -> cached device logits -> device sampler."""

    def __init__(self, vllm_config: Any, device: torch.device | str | None = None,
                 model: Any = None, max_num_reqs: int = 1024, max_prompt_len: int = 8192,
                 max_output_len: int = 8192, vocab_size: int | None = None,
                 logit_softcap: float | None = None, logit_softcap_f16: bool = False,
                 token_state: bool = True) -> None:
        """``logit_softcap``: set when ``model`` returns logits before Gemma's final soft cap;
        the sampler then applies the cap inside its launch (``logit_softcap_f16``: rounding
        each capped value to float16, as the reference stores it).  The model's logits may be
        float32, bfloat16 or float16 (sampled without a cast).  ``token_state``: keep the
        penalties' history as a per-slot token-state table on the device (``max_num_reqs`` x
        vocab words) instead of gathering id lists every step."""
        self.vllm_config = vllm_config
        self.device = torch.device(device if device is not None else "cuda")
        self.model = model
        self.sampler = Sampler(logit_softcap=logit_softcap, logit_softcap_f16=logit_softcap_f16)
        self._last_logits: torch.Tensor | None = None
        self._last_req_ids: list[str] = []
        self._max = (max_num_reqs, max_prompt_len, max_output_len)
        self._token_state = token_state
        self._vocab_size = vocab_size
        self.input_batch: InputBatch | None = None

    # -- state ---------------------------------------------------------------------------
    def _batch(self, vocab_size: int) -> InputBatch:
        if self.input_batch is None:
            self.input_batch = InputBatch(*self._max, vocab_size, self.device,
                                          token_state=self._token_state)
        elif self.input_batch.vocab_size != vocab_size:
            raise ValueError(f"vocab size changed from {self.input_batch.vocab_size} to {vocab_size}")
        return self.input_batch

    def _update_states(self, scheduler_output: Any, vocab_size: int) -> list[str]:
        batch = self._batch(vocab_size)
        for rid in getattr(scheduler_output, "finished_req_ids", ()) or ():
            batch.remove_request(rid)
        for nr in getattr(scheduler_output, "scheduled_new_reqs", ()) or ():
            batch.add_request(nr.req_id, list(nr.prompt_token_ids or []), nr.sampling_params)
        order = list(getattr(scheduler_output, "num_scheduled_tokens", {}) or {})
        if not order:
            cached = getattr(scheduler_output, "scheduled_cached_reqs", None)
            order = list(getattr(cached, "req_ids", []) or [])
            order += [nr.req_id for nr in getattr(scheduler_output, "scheduled_new_reqs", ()) or ()]
        return order

    def load_model(self) -> None:
        if self.model is None:
            raise NotImplementedError("model construction is not part of the sampling package; "
                                      "pass a model object with forward(input_ids, positions, "
                                      "scheduler_output) -> device logits")

    # -- steps -----------------------------------------------------------------------------
    def execute_model(self, scheduler_output: Any) -> None:
        """Runs the model on the scheduled requests and caches the logits (returns ``None``;
        ``sample_tokens`` produces the step's output)."""
        if self.model is None:
            return None
        try:
            vocab = self._vocab_size or getattr(self.model, "vocab_size")
            req_ids = self._update_states(scheduler_output, vocab)
            if not req_ids:
                self._last_logits, self._last_req_ids = None, []
                return None
            # inputs come from the device tables: correct even while the previous step's
            # output is still being copied to the host (async output)
            input_ids, positions = self.input_batch.decode_inputs(req_ids)
            logits = self.model.forward(input_ids, positions, scheduler_output)
            if logits.shape != (len(req_ids), vocab):
                raise ValueError(f"model returned logits {tuple(logits.shape)}, expected "
                                 f"({len(req_ids)}, {vocab})")
            self._last_logits, self._last_req_ids = logits, req_ids
            return None
        except Exception as e:
            logger.exception("execute_model failed: %s", e)
            raise

    def sample_tokens(self, grammar_output: Any, async_output: bool = False):
        """Samples the cached logits.

        The sampled ids (and logprobs) reach the host through one copy into pinned memory.
        With ``async_output`` the copy is only enqueued and an ``AsyncModelRunnerOutput`` is
        returned: its ``get_output()`` waits for the copy, so the host can schedule the next
        step while the device finishes this one (the device-side history tables are updated on
        the device either way).  The next step may be executed before ``get_output()``: its
        inputs, penalty histories and min-tokens counts come from the device-side state.
        Bad-words matching reads the host copies of the generated ids, which ``get_output()``
        appends, so a batch that uses bad words must call it before the next step samples
        (sampling raises otherwise).  ``grammar_output`` (vLLM-v1's ``GrammarOutput``) restricts
        its structured-output rows to their bitmask's tokens.
        """
        if self._last_logits is None:
            return None
        req_ids, logits = self._last_req_ids, self._last_logits
        self._last_logits = None
        batch = self.input_batch
        md = batch.make_sampling_metadata(req_ids)
        # structured output: without logprobs the grammar bitmask joins the kernel's allowed
        # mask (the result is the same as masking the logits); with logprobs the logits are
        # masked first, as vLLM-v1 does, so that the raw logprobs see the mask
        words = grammar_words(grammar_output, req_ids, logits.shape[1], logits.device)
        if words is not None:
            if md.max_num_logprobs is None:
                md.allowed_words = words
            else:
                logits = apply_grammar_words(logits.clone() if not logits.is_contiguous() else logits, words)
        out = self.sampler(logits, md)
        sampled = out.sampled_token_ids[:, 0]
        batch.append_sampled(req_ids, sampled)
        pending = AsyncModelRunnerOutput(batch, list(req_ids), sampled, out.logprobs_tensors)
        return pending if async_output else pending.get_output()

    def supported_worker_tasks(self) -> tuple[str, ...]:
        return ("generate",)

    def reset_mm_cache(self) -> None:
        pass

    def reset_encoder_cache(self) -> None:
        pass


# Drop-in name of the reference class this runner replaces (vllm_webgpu/v1/model_runner.py:54).
WebGPUModelRunner = ROCmModelRunner
