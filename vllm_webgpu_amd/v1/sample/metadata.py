"""``SamplingMetadata``: the per-step batch of sampling parameters, in vLLM-v1's shape.

The reference has no sampling metadata of its own: its runner argmaxes on the host
(``vllm_webgpu/v1/model_runner.py:145``) and leaves everything else to vLLM's sampler
(``docs/superpowers/specs/2026-06-29-vllm-webgpu-design.md:451``).  The fields below are vLLM-v1's
(``vllm/v1/sample/metadata.py``), plus ``min_p`` as a tensor (vLLM-v1 carries it inside its
built-in min-p logits processor) and ``output_token_ids_tensor``, an optional padded device copy
of ``output_token_ids`` that a persistent batch can keep resident between steps.

Conventions the kernels rely on:

* ``temperature`` is float32 ``[B]``; rows with ``temperature < 1e-5`` are greedy.  ``None``
  means every row is greedy (``all_greedy``).
* ``top_k`` int32 ``[B]`` (``<= 0`` or ``>= V`` is off), ``top_p`` / ``min_p`` float32 ``[B]``
  (``1.0`` / ``0.0`` are off).  ``None`` turns the step off for the whole batch.
* ``prompt_token_ids`` int32/int64 ``[B, P]`` padded with ``vocab_size`` (vLLM pads with V); any
  id outside ``[0, V)`` is padding.
* ``generators`` maps a row index to the ``torch.Generator`` of a seeded request; the uniforms of
  that row are drawn from it, the others from torch's default generator.
* Logits processors (vLLM-v1, applied before the penalties): ``allowed_token_ids_mask`` bool
  ``[B, V]`` with True for tokens that are *not* allowed (vLLM's convention),
  ``bad_words_token_ids`` row -> token sequences (the last token of a sequence is banned when the
  output ends with the rest of it), ``min_tokens`` row -> (minimum output length, stop token
  ids banned until it is reached), ``logit_bias`` per row (token -> bias) or None.
* ``token_state`` (this package's extension): int32 ``[R, V]`` per-request token-state table
  kept on the device by a persistent batch (bit 31: the token is in the prompt; low bits: its
  count in the output), with ``token_state_rows`` int32 ``[B]`` giving each row's table row and
  ``token_state_bits`` int32 ``[R, ceil(V/32)]`` the bitmap of its non-zero words (or None).
  When set, the penalties read it instead of ``prompt_token_ids`` / ``output_token_ids``: the
  prompt mask and output bin counts vLLM-v1 rebuilds every step, kept up to date instead.
* ``allowed_words`` (extension): int32 ``[B, ceil(V/32)]`` allowed-token bit words (bit set =
  allowed), ANDed with ``allowed_token_ids_mask``; the runner puts a step's structured-output
  grammar bitmask here.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class SamplingMetadata:
    temperature: torch.Tensor | None
    all_greedy: bool
    all_random: bool
    top_p: torch.Tensor | None
    top_k: torch.Tensor | None
    generators: dict[int, torch.Generator]
    max_num_logprobs: int | None
    no_penalties: bool
    prompt_token_ids: torch.Tensor | None
    frequency_penalties: torch.Tensor | None
    presence_penalties: torch.Tensor | None
    repetition_penalties: torch.Tensor | None
    output_token_ids: list[list[int]]
    min_p: torch.Tensor | None = None
    allowed_token_ids_mask: torch.Tensor | None = None
    bad_words_token_ids: dict[int, list[list[int]]] = field(default_factory=dict)
    output_token_ids_tensor: torch.Tensor | None = None
    output_token_lens: torch.Tensor | None = None
    min_tokens: dict[int, tuple[int, set[int]]] = field(default_factory=dict)
    logit_bias: list[dict[int, float] | None] | None = None
    token_state: torch.Tensor | None = None
    token_state_rows: torch.Tensor | None = None
    token_state_bits: torch.Tensor | None = None
    allowed_words: torch.Tensor | None = None
