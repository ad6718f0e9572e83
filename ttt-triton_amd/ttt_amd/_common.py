"""Small host-side helpers shared by the launchers."""

from __future__ import annotations

import torch

from . import _lib


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dt == torch.float16:
        return _lib.DTYPE_F16
    if dt == torch.float32:
        return _lib.DTYPE_F32
    raise ValueError(f"unsupported activation dtype {dt} (float32, bfloat16 or float16)")


def as_act(t: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """Activation in the path's dtype, contiguous (no copy when already so)."""
    return t.detach().to(dt).contiguous()


def eta_operand(eta: torch.Tensor, rule: int, dt: torch.dtype):
    """(eta as the kernels read it, the rule code to pass).  A dense eta keeps
    its own dtype when that is fp32 under 16-bit activations (TTT_ETA_DENSE_F32,
    its gradient then fp32 too), as the reference's kernels read eta in
    whatever dtype it comes; any other dense eta goes in the activation dtype.
    A learning-rate vector is fp32."""
    if rule == _lib.ETA_DENSE:
        if eta.dtype == torch.float32 and dt != torch.float32:
            return eta.detach().contiguous(), _lib.ETA_DENSE_F32
        return as_act(eta, dt), rule
    return eta.detach().to(torch.float32).contiguous(), rule


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
