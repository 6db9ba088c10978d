"""Validated sampler configuration from the environment (``envs.py``), in the reference's
pattern (``vllm_webgpu/config.py:13-75``: a dataclass with ``from_env``, checks in
``__post_init__`` that name the variable, and a cached ``get_config``)."""
from __future__ import annotations

from dataclasses import dataclass

from . import envs


@dataclass
class SamplerConfig:
    token_state: bool
    async_output: bool
    coop_wait_polls: int
    max_num_reqs: int
    debug: bool

    def __post_init__(self) -> None:
        if not (0 <= self.coop_wait_polls < 2 ** 31):
            raise ValueError(f"VLLM_WEBGPU_AMD_COOP_WAIT_POLLS={self.coop_wait_polls!r} must be in "
                             "[0, 2^31)")
        if self.max_num_reqs < 1:
            raise ValueError(f"VLLM_WEBGPU_AMD_MAX_NUM_REQS={self.max_num_reqs!r} must be >= 1")

    @classmethod
    def from_env(cls) -> "SamplerConfig":
        try:
            polls = envs.VLLM_WEBGPU_AMD_COOP_WAIT_POLLS
            reqs = envs.VLLM_WEBGPU_AMD_MAX_NUM_REQS
        except ValueError as e:
            raise ValueError(f"sampler environment: {e}") from e
        return cls(token_state=envs.VLLM_WEBGPU_AMD_TOKEN_STATE,
                   async_output=envs.VLLM_WEBGPU_AMD_ASYNC_OUTPUT, coop_wait_polls=polls,
                   max_num_reqs=reqs, debug=envs.VLLM_WEBGPU_AMD_DEBUG)

    def apply(self) -> None:
        """Hands the library its process-wide settings (the cooperative wait bound)."""
        from . import _lib

        if _lib.lib().vws_set_coop_wait_polls(self.coop_wait_polls) < 0:
            raise ValueError(_lib.last_error())


_config: SamplerConfig | None = None


def get_config() -> SamplerConfig:
    global _config
    if _config is None:
        _config = SamplerConfig.from_env()
    return _config


def reset_config() -> None:
    global _config
    _config = None
