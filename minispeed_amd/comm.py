"""Process-group view of one GPU.

This package runs the boundary step of ONE rank on ONE GPU.  The helpers
keep minispeed's names (minispeed/comm.py:22-148) and their single-process
behaviour: rank/world come from the environment when no process group exists
(so a ``FlatParamGroup`` can be built as "rank r of W" for one rank's shard),
collectives are identities, the world-1 reduce-scatter / all-gather are
copies.  Starting a multi-process job is rejected: the RCCL exchange of a
multi-GPU boundary step is not implemented in this package.
"""

from __future__ import annotations

import os

import torch
import torch.distributed as dist


class MultiGPUNotSupported(RuntimeError):
    """Raised when a job asks for more than one rank."""


def _env_int(name: str, default: int) -> int:
    try:
        return int(os.environ.get(name, default))
    except ValueError:
        return default


def resolve_backend() -> str:
    backend = os.environ.get("MINISPEED_BACKEND")
    if backend:
        return backend
    return "nccl" if torch.cuda.is_available() else "gloo"


def resolve_device() -> torch.device:
    """``MINISPEED_DEVICE`` override, else the local rank's GPU.

    The boundary kernels need a HIP device; a CPU device is rejected where
    buffers are created (flat.py), not here, so that host-only code can
    still ask which device would be used.
    """
    name = os.environ.get("MINISPEED_DEVICE")
    if name:
        dev = torch.device(name)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", min(get_local_rank(), max(torch.cuda.device_count() - 1, 0)))
        return dev
    if torch.cuda.is_available():
        return torch.device("cuda", min(get_local_rank(), torch.cuda.device_count() - 1))
    return torch.device("cpu")


def get_rank() -> int:
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank()
    return _env_int("RANK", 0)


def get_world_size() -> int:
    if dist.is_available() and dist.is_initialized():
        return dist.get_world_size()
    return _env_int("WORLD_SIZE", 1)


def get_local_rank() -> int:
    return _env_int("LOCAL_RANK", 0)


def is_distributed() -> bool:
    return dist.is_available() and dist.is_initialized() and dist.get_world_size() > 1


def init_distributed() -> None:
    """Accept a world of one; refuse anything larger."""
    if is_distributed() or get_world_size() > 1:
        raise MultiGPUNotSupported(
            f"world_size={get_world_size()}: minispeed_amd runs one rank on one GPU; "
            "the multi-GPU exchange (reduce-scatter, norm partials, all-gather) "
            "is not implemented"
        )


def barrier() -> None:
    return None


def all_reduce(tensor: torch.Tensor, op: str = "sum") -> torch.Tensor:
    return tensor


def all_reduce_flag(flag: bool) -> bool:
    return bool(flag)


def reduce_scatter(output: torch.Tensor, input_: torch.Tensor) -> torch.Tensor:
    if output.data_ptr() != input_.data_ptr():
        output.copy_(input_)
    return output


def all_gather_flat(output: torch.Tensor, local_shard: torch.Tensor) -> torch.Tensor:
    if output.data_ptr() != local_shard.data_ptr():
        output.copy_(local_shard)
    return output


def broadcast(tensor: torch.Tensor, src: int = 0) -> torch.Tensor:
    return tensor
