"""Worker: one process per MI355X, owning the device and the sampling model runner.

Mirrors the sampling-related surface of ``WebGPUWorker`` (``vllm_webgpu/v1/worker.py:58-190``):
``init_device``, ``load_model``, ``execute_model`` / ``sample_tokens`` (``:133-137``, forwarded to
the runner), ``get_supported_tasks``, ``check_health`` and ``shutdown``.  Where the reference
initialises a WebGPU adapter and a gloo process group (``:85-100``), this worker binds the
process to one ROCm device; the sampler is row-parallel and runs no collectives.
"""
from __future__ import annotations

import gc
import logging
from typing import Any

import torch

from ..config import get_config
from .model_runner import ROCmModelRunner

logger = logging.getLogger(__name__)


class ROCmWorker:
    def __init__(self, vllm_config: Any, local_rank: int = 0, rank: int = 0,
                 distributed_init_method: str = "", is_driver_worker: bool = False,
                 model: Any = None, **runner_kwargs: Any) -> None:
        self.vllm_config = vllm_config
        self.local_rank = local_rank
        self.rank = rank
        self.distributed_init_method = distributed_init_method
        self.is_driver_worker = is_driver_worker
        self._model = model
        self._runner_kwargs = runner_kwargs
        self.device: torch.device | None = None
        self.model_runner: ROCmModelRunner | None = None

    def init_device(self) -> None:
        if not torch.cuda.is_available():
            raise RuntimeError("no ROCm device is visible to this process")
        self.device = torch.device(f"cuda:{self.local_rank}")
        torch.cuda.set_device(self.device)
        # the sampler's settings from the environment (VLLM_WEBGPU_AMD_*); explicit runner
        # arguments take precedence
        cfg = get_config()
        cfg.apply()
        kwargs = dict(token_state=cfg.token_state, max_num_reqs=cfg.max_num_reqs)
        kwargs.update(self._runner_kwargs)
        self._async_output = cfg.async_output
        self.model_runner = ROCmModelRunner(self.vllm_config, self.device, self._model, **kwargs)

    def load_model(self) -> None:
        self.model_runner.load_model()

    def execute_model(self, scheduler_output: Any) -> Any:
        return self.model_runner.execute_model(scheduler_output)

    def sample_tokens(self, grammar_output: Any) -> Any:
        return self.model_runner.sample_tokens(grammar_output,
                                               async_output=getattr(self, "_async_output", False))

    def get_model(self) -> Any:
        return self.model_runner.model

    def get_supported_tasks(self) -> tuple:
        return self.model_runner.supported_worker_tasks()

    def check_health(self) -> None:
        """Round-trips a one-element kernel through the device queue."""
        if self.device is None:
            raise RuntimeError("device not initialized")
        try:
            x = torch.ones(1, device=self.device)
            if float((x + x).item()) != 2.0:
                raise RuntimeError("device returned a wrong result")
        except Exception as e:
            raise RuntimeError(f"ROCm device health check failed: {e}") from e

    def shutdown(self) -> None:
        self.model_runner = None
        gc.collect()
        logger.info("ROCm worker shutdown complete")


# Drop-in name of the reference class this worker replaces (vllm_webgpu/v1/worker.py:58).
WebGPUWorker = ROCmWorker
