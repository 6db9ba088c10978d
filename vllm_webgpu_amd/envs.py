"""Environment variables of the MI355X sampler, read lazily like the reference plugin's own
(``vllm_webgpu/envs.py:12-18``: a name -> reader table behind a module ``__getattr__``).

* ``VLLM_WEBGPU_AMD_TOKEN_STATE`` (bool, default 1): the runner keeps the penalties' history as
  a per-slot token-state table on the device instead of gathering id lists every step.
* ``VLLM_WEBGPU_AMD_ASYNC_OUTPUT`` (bool, default 0): ``sample_tokens`` returns an
  ``AsyncModelRunnerOutput`` whose device-to-host copy is still in flight.
* ``VLLM_WEBGPU_AMD_COOP_WAIT_POLLS`` (int, default 1048576): bound of a top-p row's wait for
  the shared passes other workgroups run (``vws_set_coop_wait_polls``).
* ``VLLM_WEBGPU_AMD_MAX_NUM_REQS`` (int, default 1024): request slots of the persistent batch.
* ``VLLM_WEBGPU_AMD_DEBUG`` (bool, default 0): check every launch's status synchronously.
"""
from __future__ import annotations

import os
from collections.abc import Callable
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    VLLM_WEBGPU_AMD_TOKEN_STATE: bool = True
    VLLM_WEBGPU_AMD_ASYNC_OUTPUT: bool = False
    VLLM_WEBGPU_AMD_COOP_WAIT_POLLS: int = 1 << 20
    VLLM_WEBGPU_AMD_MAX_NUM_REQS: int = 1024
    VLLM_WEBGPU_AMD_DEBUG: bool = False


def _flag(name: str, default: str) -> bool:
    return os.getenv(name, default).strip().lower() in ("1", "true", "yes", "on")


environment_variables: dict[str, Callable[[], Any]] = {
    "VLLM_WEBGPU_AMD_TOKEN_STATE": lambda: _flag("VLLM_WEBGPU_AMD_TOKEN_STATE", "1"),
    "VLLM_WEBGPU_AMD_ASYNC_OUTPUT": lambda: _flag("VLLM_WEBGPU_AMD_ASYNC_OUTPUT", "0"),
    "VLLM_WEBGPU_AMD_COOP_WAIT_POLLS": lambda: int(os.getenv("VLLM_WEBGPU_AMD_COOP_WAIT_POLLS", str(1 << 20))),
    "VLLM_WEBGPU_AMD_MAX_NUM_REQS": lambda: int(os.getenv("VLLM_WEBGPU_AMD_MAX_NUM_REQS", "1024")),
    "VLLM_WEBGPU_AMD_DEBUG": lambda: _flag("VLLM_WEBGPU_AMD_DEBUG", "0"),
}


def __getattr__(name: str) -> Any:
    if name in environment_variables:
        return environment_variables[name]()
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
