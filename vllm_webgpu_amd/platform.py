"""vLLM out-of-tree platform hook that routes the engine to the MI355X worker.

Mirrors ``WebGPUPlatform`` (``vllm_webgpu/platform.py:52-147``): device queries and
``check_and_update_config``, which points ``worker_cls`` at this package's worker (the reference
routes to ``vllm_webgpu.v1.worker.WebGPUWorker`` at ``:106-113``).  Device queries answer for
the ROCm device torch sees; pinned host memory is available (the reference disables it,
``:128-130``) and is used for the sampled-id readback.
"""
from __future__ import annotations

from typing import Any

try:  # pragma: no cover - vLLM is not installed in the build container
    from vllm.platforms.interface import Platform as _Platform
    from vllm.platforms.interface import PlatformEnum as _PlatformEnum
except ImportError:
    _Platform = object

    class _PlatformEnum:  # type: ignore[no-redef]
        OOT = "OOT"

WORKER_CLS = "vllm_webgpu_amd.v1.worker.ROCmWorker"


class MI355XPlatform(_Platform):
    _enum = _PlatformEnum.OOT
    device_name: str = "cuda"
    device_type: str = "cuda"
    dispatch_key: str = "CUDA"

    @classmethod
    def is_available(cls) -> bool:
        try:
            import torch
            return torch.cuda.is_available() and "gfx950" in torch.cuda.get_device_properties(0).gcnArchName
        except Exception:
            return False

    @classmethod
    def get_device_name(cls, device_id: int = 0) -> str:
        import torch
        return torch.cuda.get_device_name(device_id)

    @classmethod
    def get_device_count(cls) -> int:
        import torch
        return torch.cuda.device_count()

    @classmethod
    def get_device_total_memory(cls, device_id: int = 0) -> int:
        import torch
        return torch.cuda.get_device_properties(device_id).total_memory

    @classmethod
    def check_and_update_config(cls, vllm_config: Any) -> None:
        pc = vllm_config.parallel_config
        if pc.worker_cls == "auto":
            pc.worker_cls = WORKER_CLS
        pc.distributed_executor_backend = "uni"

    @classmethod
    def is_pin_memory_available(cls) -> bool:
        return True

    @classmethod
    def set_device(cls, device_id: int) -> None:
        import torch
        torch.cuda.set_device(device_id)

    @classmethod
    def current_device(cls) -> int:
        import torch
        return torch.cuda.current_device()

    @classmethod
    def synchronize(cls, device_id: int = 0) -> None:
        import torch
        torch.cuda.synchronize(device_id)


# Drop-in name of the reference class this platform replaces (vllm_webgpu/platform.py:52).
WebGPUPlatform = MI355XPlatform
