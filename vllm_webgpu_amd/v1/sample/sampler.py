"""``Sampler``: vLLM-v1's sampling layer as one call into the gfx950 library.

Reference anchors: the reference samples greedily on the host
(``vllm_webgpu/v1/model_runner.py:139-159``, ``logits.argmax(axis=-1)``) and otherwise defers to
vLLM's CPU sampler (``docs/superpowers/specs/2026-06-29-vllm-webgpu-design.md:451``).  This class
keeps vLLM-v1's ``Sampler.forward(logits, sampling_metadata) -> SamplerOutput`` signature and its
order of operations -- raw logprobs of the unprocessed logits, logits processors (allowed-token
mask, bad words, min-tokens, logit bias), penalties, greedy argmax of the processed logits,
temperature, min-p, top-k, top-p, exponential race, logprob gather -- but runs all of it in a
single stream-ordered kernel launch (``vws_sample``) on device-resident logits; only the sparse
processor lists (bad-word matches, min-tokens bans, biases) are built on the host.

Random rows race with the key ``p / (-ln u)``: an exponential race, as vLLM's
``random_sample`` (``probs / q.exponential_()``).  The uniforms ``u`` are generated inside the
launch (Philox-4x32-10, only where a token races), so no ``[B, V]`` tensor is drawn or read:
from one 64-bit key per launch, drawn from torch's default generator and passed by value,
when no request is seeded; otherwise from one key per row and step (the request's own stream
for seeded rows), uploaded with one copy.

There is no host fallback: without the HIP library, or for logits that are not on a ROCm device,
``forward`` raises.
"""
from __future__ import annotations

import numpy as np
import torch

from ... import ops
from ..outputs import LogprobsTensors, SamplerOutput
from .metadata import SamplingMetadata

_SEED_LO, _SEED_HI = -2 ** 63, 2 ** 63 - 1
_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(x: np.ndarray) -> np.ndarray:
    """SplitMix64's output function (Steele, Lea and Flood, OOPSLA 2014) on uint64 states."""
    with np.errstate(over="ignore"):
        z = x.astype(np.uint64)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


class KeyStream:
    """A seeded request's per-step race keys: step n's key is SplitMix64 of
    ``seed + (n + 1) * 0x9E3779B97F4A7C15``, so the request draws the same keys, and samples
    the same tokens, whenever it runs again with its seed.  Stands in for a ``torch.Generator``
    in ``SamplingMetadata.generators`` so that a whole batch's keys come from one host-side
    computation (``draw_seeds``)."""

    _GOLDEN = 0x9E3779B97F4A7C15

    def __init__(self, seed: int) -> None:
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.step = 0

    @staticmethod
    def keys(seeds: np.ndarray, steps: np.ndarray) -> np.ndarray:
        """int64 keys of the given (seed, step) pairs."""
        with np.errstate(over="ignore"):
            st = seeds.astype(np.uint64) + (steps.astype(np.uint64) + np.uint64(1)) * np.uint64(KeyStream._GOLDEN)
        return splitmix64(st).view(np.int64)

    def next_key(self) -> int:
        k = int(self.keys(np.array([self.seed], np.uint64), np.array([self.step], np.uint64))[0])
        self.step += 1
        return k


class SeedStaging:
    """Reusable buffers for ``draw_seeds``: a ring of pinned host buffers and one device buffer,
    so that a step's keys take no allocation.  A host buffer is written again only once the
    copy that last read it has completed (an event per buffer); the device buffer is rewritten
    by the next step's copy, which the stream orders after this step's kernel.  One staging
    object per stream."""

    RING = 4

    def __init__(self) -> None:
        self.cap = 0
        self.host = self.dev = None
        self.events = []
        self.i = 0

    def acquire(self, B: int, device: torch.device):
        if B > self.cap or self.dev is None or self.dev.device != device:
            self.cap = max(B, 2 * self.cap, 64)
            self.host = torch.empty((self.RING, self.cap), dtype=torch.int64, pin_memory=True)
            self.dev = torch.empty(self.cap, dtype=torch.int64, device=device)
            # (waiting on an event never recorded returns at once)
            self.events = [torch.cuda.Event() for _ in range(self.RING)]
        self.i = (self.i + 1) % self.RING
        self.events[self.i].synchronize()
        return self.host[self.i, :B], self.dev[:B]

    def copied(self) -> None:
        self.events[self.i].record()


def draw_seeds(B: int, generators: dict, device: torch.device,
               staging: SeedStaging | None = None) -> torch.Tensor:
    """int64 ``[B]`` keys of the race's generated uniforms, one fresh draw per row and step: row
    ``i`` draws from ``generators[i]`` if present (a seeded request samples the same tokens
    again), the others from torch's default CPU generator.  ``KeyStream`` entries (the
    persistent batch's seeded requests) are computed together on the host; a ``torch.Generator``
    entry draws from its own stream.  One host-to-device copy; with ``staging`` (device
    tensors only) no allocation, and the returned tensor is the staging's device buffer, valid
    until the next draw on it."""
    use = staging is not None and device.type == "cuda"
    if use:
        keys, dev_keys = staging.acquire(B, device)
        torch.randint(_SEED_LO, _SEED_HI, (B,), dtype=torch.int64, out=keys)
    else:
        keys = torch.randint(_SEED_LO, _SEED_HI, (B,), dtype=torch.int64)
    ks = [(i, g) for i, g in generators.items() if isinstance(g, KeyStream)]
    if ks:
        rows = np.array([i for i, _ in ks], np.int64)
        seeds = np.array([g.seed for _, g in ks], np.uint64)
        steps = np.array([g.step for _, g in ks], np.uint64)
        keys[torch.from_numpy(rows)] = torch.from_numpy(KeyStream.keys(seeds, steps))
        for _, g in ks:
            g.step += 1
    for i, g in generators.items():
        if not isinstance(g, KeyStream):
            keys[i] = torch.randint(_SEED_LO, _SEED_HI, (1,), dtype=torch.int64,
                                    device=g.device, generator=g)[0].cpu()
    if use:
        dev_keys.copy_(keys, non_blocking=True)
        staging.copied()
        return dev_keys
    if device.type == "cuda":
        keys = keys.pin_memory()
    return keys.to(device, non_blocking=True)


def pad_output_ids(output_token_ids: list[list[int]], vocab_size: int,
                   device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """Packs ragged output histories into int32 ``[B, W]`` padded with ``vocab_size`` (+ lengths)."""
    B = len(output_token_ids)
    W = max((len(t) for t in output_token_ids), default=0)
    host = torch.full((B, max(W, 1)), vocab_size, dtype=torch.int32,
                      pin_memory=torch.cuda.is_available())
    lens = torch.empty(B, dtype=torch.int32, pin_memory=torch.cuda.is_available())
    for i, t in enumerate(output_token_ids):
        if t:
            host[i, :len(t)] = torch.as_tensor(t, dtype=torch.int32)
        lens[i] = len(t)
    return host.to(device, non_blocking=True), lens.to(device, non_blocking=True)


def processor_lists(m: SamplingMetadata, B: int, V: int):
    """Host-side (ids, vals, lens): int32/float32 [B, W] of the sparse logits processors and
    int32 [B] entries per row, or None.  The lengths let rows without an entry keep their
    paths (a row counts as carrying processors only when its length is non-zero).

    Bad words follow vLLM-v1's ``apply_bad_words``: a sequence bans its last token when the
    row's output ends with the rest of it (single-token sequences always).  Min-tokens bans the
    stop tokens while the output is shorter than the minimum.  Logit bias adds its value.
    Padding ids are V.
    """
    if not m.bad_words_token_ids and not m.min_tokens and not (m.logit_bias and any(m.logit_bias)):
        return None  # the common case, without a pass over the rows
    rows: list[list[tuple[int, float]]] = [[] for _ in range(B)]
    for i, words in (m.bad_words_token_ids or {}).items():
        past = m.output_token_ids[i] if i < len(m.output_token_ids) else []
        for seq in words:
            if not seq or len(seq) > len(past) + 1:
                continue
            prefix = list(seq[:-1])
            if not prefix or list(past[-len(prefix):]) == prefix:
                rows[i].append((int(seq[-1]), float("-inf")))
    for i, (min_toks, stop_ids) in (m.min_tokens or {}).items():
        past = m.output_token_ids[i] if i < len(m.output_token_ids) else []
        if len(past) < min_toks:
            rows[i].extend((int(t), float("-inf")) for t in stop_ids)
    for i, bias in enumerate(m.logit_bias or []):
        if bias:
            rows[i].extend((int(t), float(b)) for t, b in bias.items())
    width = max((len(r) for r in rows), default=0)
    if width == 0:
        return None
    ids = torch.full((B, width), V, dtype=torch.int32)
    vals = torch.zeros((B, width), dtype=torch.float32)
    lens = torch.tensor([len(r) for r in rows], dtype=torch.int32)
    for i, r in enumerate(rows):
        if r:
            ids[i, :len(r)] = torch.tensor([t for t, _ in r], dtype=torch.int32)
            vals[i, :len(r)] = torch.tensor([v for _, v in r], dtype=torch.float32)
    return ids, vals, lens


class Sampler:
    """vLLM-v1 ``Sampler`` facade over ``vws_sample``."""

    def __init__(self, logprobs_mode: str = "raw_logprobs",
                 logit_softcap: float | None = None, logit_softcap_f16: bool = False) -> None:
        """``logit_softcap``: Gemma's final soft cap, fused into the sampling launch, for models
        whose forward returns the lm_head output before the cap (reference:
        ``vllm_webgpu/models/gemma4.py:158-163``).  The capped logits are then the model's
        output for everything that follows, raw logprobs included.  ``logit_softcap_f16``:
        each capped value is rounded to float16, as the reference's shader stores it
        (``shaders/gemma/logit_softcap.wgsl:28``).  Logits may be float32, bfloat16 or float16."""
        if logprobs_mode != "raw_logprobs":
            raise NotImplementedError(
                f"logprobs_mode {logprobs_mode!r}: only 'raw_logprobs' (log-softmax of the "
                "unprocessed logits) is computed by the device sampler")
        if logit_softcap is not None and not (0.0 < float(logit_softcap) < float("inf")):
            raise ValueError(f"logit_softcap must be a positive finite number (got {logit_softcap})")
        self.logprobs_mode = logprobs_mode
        self.logit_softcap = logit_softcap
        self.logit_softcap_f16 = bool(logit_softcap_f16)
        self._seeds = SeedStaging()

    def __call__(self, logits: torch.Tensor, sampling_metadata: SamplingMetadata) -> SamplerOutput:
        return self.forward(logits, sampling_metadata)

    def forward(self, logits: torch.Tensor, sampling_metadata: SamplingMetadata) -> SamplerOutput:
        m = sampling_metadata
        if logits.dim() != 2:
            raise ValueError(f"logits must be [num_reqs, vocab] (got {tuple(logits.shape)})")
        B, V = logits.shape
        dev = logits.device

        temperature = None if m.all_greedy else m.temperature
        seeds = key = None
        if temperature is not None:
            if m.generators:
                seeds = draw_seeds(B, m.generators, dev, self._seeds)
            else:
                # no seeded request: one key for the launch, from torch's default generator,
                # passed by value (row r draws as with that seed and offset r)
                key = int(torch.randint(_SEED_LO, _SEED_HI, (1,), dtype=torch.int64))

        penalties = {}
        if not m.no_penalties and m.token_state is not None:
            penalties = dict(repetition_penalty=m.repetition_penalties,
                             presence_penalty=m.presence_penalties,
                             frequency_penalty=m.frequency_penalties,
                             token_state=m.token_state, token_state_rows=m.token_state_rows,
                             token_state_bits=m.token_state_bits)
        elif not m.no_penalties:
            out_ids, out_lens = m.output_token_ids_tensor, m.output_token_lens
            if out_ids is None and any(m.output_token_ids):
                out_ids, out_lens = pad_output_ids(m.output_token_ids, V, dev)
            penalties = dict(repetition_penalty=m.repetition_penalties,
                             presence_penalty=m.presence_penalties,
                             frequency_penalty=m.frequency_penalties,
                             prompt_ids=m.prompt_token_ids, output_ids=out_ids,
                             output_lens=out_lens)

        processors = {}
        if m.allowed_token_ids_mask is not None:
            processors["allowed_mask"] = ops.pack_allowed(~m.allowed_token_ids_mask.to(dev, torch.bool))
        if m.allowed_words is not None:
            w = m.allowed_words.to(dev, torch.int32)
            processors["allowed_mask"] = (w if "allowed_mask" not in processors
                                          else processors["allowed_mask"] & w)
        adj = processor_lists(m, B, V)
        if adj is not None:
            ids, vals, lens = adj
            processors.update(adjust_ids=ids.to(dev, non_blocking=True),
                              adjust_vals=vals.to(dev, non_blocking=True),
                              adjust_lens=lens.to(dev, non_blocking=True))

        res = ops.sample(logits, temperature=temperature, top_k=m.top_k, top_p=m.top_p,
                         min_p=m.min_p, rng_seeds=seeds, rng_key=key,
                         num_logprobs=m.max_num_logprobs,
                         logit_softcap=self.logit_softcap,
                         logit_softcap_f16=self.logit_softcap_f16, **penalties, **processors)
        lp = None
        if m.max_num_logprobs is not None:
            lp = LogprobsTensors(res.logprob_ids, res.logprob_vals, res.logprob_ranks)
        return SamplerOutput(sampled_token_ids=res.sampled.unsqueeze(-1), logprobs_tensors=lp)
