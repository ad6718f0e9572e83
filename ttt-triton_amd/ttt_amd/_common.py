"""Small host-side helpers shared by the launchers."""

from __future__ import annotations

import torch

from . import _lib


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dt == torch.float32:
        return _lib.DTYPE_F32
    raise ValueError(f"unsupported activation dtype {dt} (float32 or bfloat16)")


def as_act(t: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """Activation in the path's dtype, contiguous (no copy when already so)."""
    return t.detach().to(dt).contiguous()


def check_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    if dev.type != "cuda":
        raise ValueError("the TTT HIP path needs GPU tensors (device 'cuda')")
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, got {t.device}")
    return dev


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def stream_of(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream
