"""vLLM-v1 output containers of the sampling step.

The reference imports ``SamplerOutput`` and ``ModelRunnerOutput`` from ``vllm.v1.outputs``
(``vllm_webgpu/v1/model_runner.py:8-19``) and builds them at ``model_runner.py:146-159``.  When
vLLM is importable the same classes are used here; otherwise these dataclasses stand in with the
vLLM-v1 field names and shapes:

* ``SamplerOutput.sampled_token_ids``: int32 ``[B, 1]`` device tensor;
* ``LogprobsTensors``: ``logprob_token_ids`` int32 ``[B, L+1]`` (the sampled id first, then the
  top-L ids), ``logprobs`` float32 ``[B, L+1]``, ``selected_token_ranks`` int32 ``[B]``;
* ``LogprobsLists``: the host-side lists the engine core ships to the front end;
* ``ModelRunnerOutput``: per-request results keyed by ``req_ids`` / ``req_id_to_index``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, NamedTuple

import torch

try:  # pragma: no cover - vLLM is not installed in the build container
    from vllm.v1.outputs import (LogprobsLists, LogprobsTensors, ModelRunnerOutput,
                                 SamplerOutput)
    HAVE_VLLM = True
except ImportError:
    HAVE_VLLM = False

    class LogprobsLists(NamedTuple):  # type: ignore[no-redef]
        logprob_token_ids: list[list[int]]   # [B][L+1]
        logprobs: list[list[float]]          # [B][L+1]
        sampled_token_ranks: list[int]       # [B]

        def slice(self, start: int, end: int) -> "LogprobsLists":
            return LogprobsLists(self.logprob_token_ids[start:end], self.logprobs[start:end],
                                 self.sampled_token_ranks[start:end])

    class LogprobsTensors(NamedTuple):  # type: ignore[no-redef]
        logprob_token_ids: torch.Tensor      # int32 [B, L+1]
        logprobs: torch.Tensor               # float32 [B, L+1]
        selected_token_ranks: torch.Tensor   # int32 [B]

        def tolists(self) -> LogprobsLists:
            return LogprobsLists(self.logprob_token_ids.tolist(), self.logprobs.tolist(),
                                 self.selected_token_ranks.tolist())

        @staticmethod
        def empty_cpu(num_positions: int, num_tokens_per_position: int) -> "LogprobsTensors":
            ids = torch.empty((num_positions, num_tokens_per_position), dtype=torch.int32)
            vals = torch.empty_like(ids, dtype=torch.float32)
            ranks = torch.empty(num_positions, dtype=torch.int32)
            return LogprobsTensors(ids, vals, ranks)

    @dataclass
    class SamplerOutput:  # type: ignore[no-redef]
        sampled_token_ids: torch.Tensor            # int32 [B, 1]
        logprobs_tensors: LogprobsTensors | None

    @dataclass
    class ModelRunnerOutput:  # type: ignore[no-redef]
        req_ids: list[str]
        req_id_to_index: dict[str, int]
        sampled_token_ids: list[list[int]] = field(default_factory=list)
        logprobs: LogprobsLists | None = None
        prompt_logprobs_dict: dict[str, Any] = field(default_factory=dict)
        pooler_output: list[Any] = field(default_factory=list)
        num_nans_in_logits: dict[str, int] | None = None

__all__ = ["HAVE_VLLM", "LogprobsLists", "LogprobsTensors", "ModelRunnerOutput", "SamplerOutput"]
