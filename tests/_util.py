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
