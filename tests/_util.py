"""Shared helpers for the parity tests."""

from __future__ import annotations

import torch

from oracle import ttt_oracle as O


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.detach().double().cpu() - b.detach().double().cpu()).abs().max())


def to_dev(d: dict, device="cuda") -> dict:
    return {k: v.to(device) for k, v in d.items()}


def eta_own_dtype(d: dict, dt: torch.dtype) -> dict:
    """Under fp16 activations the dense eta stays fp32 (the kernels then read
    it and write its gradient in fp32): on these unnormalised N(0, 1) inputs
    the eta gradient reaches 6e4-1.2e5, past fp16's largest value 65504."""
    if dt == torch.float16:
        d["eta"] = d["eta"].float()
    return d


def oracle_linear_grads(d: dict, dout: torch.Tensor, G: int, dtype=torch.float64):
    """Autograd of the oracle's ttt_linear, inputs upcast to `dtype`.
    dout is [B,H,NC,K,F]; returns dict of grads in [B,H,...] layouts + out."""
    names = ["XK", "XQ", "XV", "eta", "ln_w", "ln_b", "W1", "b1"]
    args = {n: d[n].detach().cpu().to(dtype).requires_grad_(True) for n in names}
    out = O.ttt_linear(*[args[n] for n in names], G)
    out.backward(dout.detach().cpu().to(dtype).permute(0, 2, 3, 1, 4))
    res = {"out": out.detach().permute(0, 3, 1, 2, 4)}
    res.update({"d" + n: args[n].grad for n in names})
    return res


def oracle_mlp_grads(d: dict, dout: torch.Tensor, G: int, dtype=torch.float64):
    names = ["XK", "XQ", "XV", "eta", "ln_w", "ln_b", "W1", "b1", "W2", "b2"]
    args = {n: d[n].detach().cpu().to(dtype).requires_grad_(True) for n in names}
    out = O.ttt_mlp(*[args[n] for n in names], G)
    out.backward(dout.detach().cpu().to(dtype).permute(0, 2, 3, 1, 4))
    res = {"out": out.detach().permute(0, 3, 1, 2, 4)}
    res.update({"d" + n: args[n].grad for n in names})
    return res


# fp32 parity bar: the required max-abs 1e-4, or, for a tensor whose own
# fp32 evaluation is less exact than that (the eta gradient reaches 1e4 on
# unnormalised N(0,1) inputs), C_FP32 times the error of the oracle run in fp32
# against the oracle in fp64 on the same inputs.  The kernels' fp32 error is
# 1-2x the fp32 oracle's (different summation orders, the same precision).
FP32_ATOL = 1e-4
C_FP32 = 8.0


def fp32_bound(ref64: torch.Tensor, ref32: torch.Tensor) -> float:
    return max(FP32_ATOL, C_FP32 * max_abs(ref32, ref64))
