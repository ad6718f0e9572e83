"""CPU oracle for the TTT-Linear / TTT-MLP mini-batch inner loop.

TEST INFRASTRUCTURE ONLY.  This module is a plain eager-PyTorch (CPU)
restatement of the reference's ops path.  It is imported by `tests/`, by
`__graft_entry__.smoke()` and by the `cpu_baseline` leg of `bench.py`, and
there only as the checker / the timed CPU baseline.  The product path
(`ttt-triton_amd/`) never imports it.

What it restates (reference file:line):
  ln_fwd             ops/ttt_utils.py:4-18      eps 1e-8, biased variance
  ln_fused_l2_bwd    ops/ttt_utils.py:21-48     d/dx of 0.5*||LN(x)-t||^2
  gelu_bwd           ops/ttt_utils.py:51-54     tanh-GELU derivative (ops constants)
  gelu_tanh          ops/ttt_mlp.py:31          F.gelu(approximate="tanh")
  linear_mini_batch  ops/ttt_linear.py:8-54     dual form, full KxK eta, no tril
  mlp_mini_batch     ops/ttt_mlp.py:9-67        dual form for both layers
  scan               utils.py:126-161           carry loop, per-group checkpoint
  ttt_linear         ops/ttt_linear.py:57-84    [B,H,NC,K,F] -> [B,NC,K,H,F]
  ttt_mlp            ops/ttt_mlp.py:70-99
  cached_readout     kernels/mlp_cached_readout.py:88-109,143 semantics with the
                     (b,h) indexing the reference kernel drops (its out[0,0] race)
  memo_combine       ttt_layer.py:506-561 (softmax gates over segment summaries,
                     cached readouts of the memo states), with correct (b,h)
                     indexing of the cached readouts
  side outputs       checkpoints = state entering mini-batch k*G
                     (kernels/linear_forward.py:55-73, kernels/mlp_forward.py:84-117);
                     memo = state after mini-batch s*M (kernels/mlp_forward.py:193-226);
                     W_last = final state (kernels/linear_forward.py:147-148)
  eta builders       ttt_layer.py:151-163,306-309 (row-constant "layer" eta) and the
                     causal variant eta[i,j] = lr[j]/(i+1) for j<=i (eta_from_lr, make_eta)
  inputs             seeded generator in the order XQ, XK, XV, u, W1, W2, dOut

How each function is pinned (tests/test_oracle.py):
  ln_fwd            == torch.nn.functional.layer_norm (library routine)
  ln_fused_l2_bwd   == autograd of 0.5*||layer_norm(x)-t||^2 (closed form)
  gelu_bwd          == autograd of F.gelu(tanh) (to the constants' 1e-9 difference)
  mini-batch steps  == brute-force per-token primal update (W_i = W - sum_j eta_ij x_j^T g_j);
                       row-constant eta == primal form; W_last closed form
  scan              forward invariant to the checkpoint group size
  backward          autograd of this restatement == fp64 finite differences (gradcheck)
  cached_readout    == mlp_mini_batch readout with eta = 0 (no update), eps 1e-8
  memo_combine      one segment == identity; XU = 0 gives the uniform average of
                    XQW and the cached readouts (closed form); identical memo states
                    with XQW = their readout leave the output unchanged (convex
                    combination); gradients == fp64 finite differences
  side outputs      checkpoints / memo / W_last == states of an independent step loop
There is no reference-held golden vector for this path (the reference ships no
tests or fixtures), so parity is pinned only by the checks above.
"""

from __future__ import annotations

import math
from typing import Callable, Dict, Optional

import torch
import torch.nn.functional as F

LN_EPS = 1e-8  # ops/ttt_utils.py:4,21


# ----------------------------------------------------------------------------
# math helpers (ops/ttt_utils.py)
# ----------------------------------------------------------------------------

def ln_fwd(x, gamma, beta, eps: float = LN_EPS):
    """LayerNorm over the last dim, biased variance.  ops/ttt_utils.py:4-18."""
    mu = x.mean(dim=-1, keepdim=True)
    var = x.var(dim=-1, keepdim=True, unbiased=False)
    std = torch.sqrt(var + eps)
    return gamma * ((x - mu) / std) + beta


def ln_fused_l2_bwd(x, target, gamma, beta, eps: float = LN_EPS):
    """Gradient wrt x of 0.5*||gamma*xhat+beta - target||^2.  ops/ttt_utils.py:21-48."""
    D = x.shape[-1]
    mu = x.mean(dim=-1, keepdim=True)
    var = x.var(dim=-1, keepdim=True, unbiased=False)
    std = torch.sqrt(var + eps)
    x_hat = (x - mu) / std
    y = gamma * x_hat + beta
    grad_x_hat = (y - target) * gamma
    return (
        (1.0 / D)
        * (
            D * grad_x_hat
            - grad_x_hat.sum(dim=-1, keepdim=True)
            - x_hat * (grad_x_hat * x_hat).sum(dim=-1, keepdim=True)
        )
        / std
    )


def gelu_bwd(x):
    """tanh-GELU derivative with the ops path's constants.  ops/ttt_utils.py:51-54."""
    t = torch.tanh(0.79788456 * x * (1 + 0.044715 * x * x))
    return 0.5 * x * ((1 - t * t) * (0.79788456 + 0.1070322243 * x * x)) + 0.5 * (1 + t)


def gelu_tanh(x):
    """ops/ttt_mlp.py:31 (F.gelu with the tanh approximation)."""
    return F.gelu(x, approximate="tanh")


# ----------------------------------------------------------------------------
# one mini-batch (dual form, general KxK eta)
# ----------------------------------------------------------------------------

def linear_mini_batch(params: Dict[str, torch.Tensor], inputs: Dict[str, torch.Tensor], eps: float = LN_EPS):
    """One TTT-Linear mini-batch.  ops/ttt_linear.py:8-54.

    params: W1_states [B,H,F,F], b1_states [B,H,1,F], ttt_norm_weight/bias [H,F]
    inputs: XQ, XK, XV [B,H,K,F], eta [B,H,K,K]
    """
    W1, b1 = params["W1_states"], params["b1_states"]
    ln_w, ln_b = params["ttt_norm_weight"], params["ttt_norm_bias"]
    XQ, XV, XK, eta = inputs["XQ"], inputs["XV"], inputs["XK"], inputs["eta"]
    H, Fd = XQ.size(1), XQ.size(-1)
    g = ln_w.reshape(H, 1, Fd)
    bt = ln_b.reshape(H, 1, Fd)

    Z1 = XK @ W1 + b1
    grad = ln_fused_l2_bwd(Z1, XV - XK, g, bt, eps)
    attn = XQ @ XK.transpose(-2, -1)
    b1_bar = b1 - eta @ grad
    Z1_bar = XQ @ W1 - (eta * attn) @ grad + b1_bar

    last = eta[:, :, -1, :, None]
    W1_last = W1 - (last * XK).transpose(-1, -2) @ grad
    b1_last = b1 - torch.sum(last * grad, dim=-2, keepdim=True)

    out = XQ + ln_fwd(Z1_bar, g, bt, eps)
    new = dict(params)
    new["W1_states"], new["b1_states"] = W1_last, b1_last
    return new, out


def mlp_mini_batch(params: Dict[str, torch.Tensor], inputs: Dict[str, torch.Tensor], eps: float = LN_EPS):
    """One TTT-MLP mini-batch.  ops/ttt_mlp.py:9-67.

    params: W1_states [B,H,F,FF], b1_states [B,H,1,FF], W2_states [B,H,FF,F],
            b2_states [B,H,1,F], ttt_norm_weight/bias [H,F]
    """
    W1, b1 = params["W1_states"], params["b1_states"]
    W2, b2 = params["W2_states"], params["b2_states"]
    ln_w, ln_b = params["ttt_norm_weight"], params["ttt_norm_bias"]
    XQ, XV, XK, eta = inputs["XQ"], inputs["XV"], inputs["XK"], inputs["eta"]
    H, Fd = XQ.size(1), XQ.size(-1)
    g = ln_w.reshape(H, 1, Fd)
    bt = ln_b.reshape(H, 1, Fd)

    Z1 = XK @ W1 + b1
    X2 = gelu_tanh(Z1)
    Z2 = X2 @ W2 + b2
    grad2 = ln_fused_l2_bwd(Z2, XV - XK, g, bt, eps)
    grad1 = grad2 @ W2.transpose(-2, -1) * gelu_bwd(Z1)

    attn1 = XQ @ XK.transpose(-2, -1)
    b1_bar = b1 - eta @ grad1
    Z1_bar = XQ @ W1 - (eta * attn1) @ grad1 + b1_bar
    X2_bar = gelu_tanh(Z1_bar)

    attn2 = X2_bar @ X2.transpose(-2, -1)
    b2_bar = b2 - eta @ grad2
    Z2_bar = X2_bar @ W2 - (eta * attn2) @ grad2 + b2_bar

    last = eta[:, :, -1, :, None]
    W1_last = W1 - (last * XK).transpose(-1, -2) @ grad1
    b1_last = b1 - torch.sum(last * grad1, dim=-2, keepdim=True)
    W2_last = W2 - (last * X2).transpose(-1, -2) @ grad2
    b2_last = b2 - torch.sum(last * grad2, dim=-2, keepdim=True)

    out = XQ + ln_fwd(Z2_bar, g, bt, eps)
    new = dict(params)
    new["W1_states"], new["b1_states"] = W1_last, b1_last
    new["W2_states"], new["b2_states"] = W2_last, b2_last
    return new, out


# ----------------------------------------------------------------------------
# scan driver (utils.py:126-161)
# ----------------------------------------------------------------------------

def scan(f: Callable, init, xs: Dict[str, torch.Tensor], checkpoint_group: int = 0,
         on_step: Optional[Callable[[int, dict], None]] = None):
    """Sequential carry over dim 0 of every tensor in `xs`.  utils.py:126-161.

    With checkpoint_group > 0 each group runs under torch.utils.checkpoint
    (use_reentrant=False), as the reference does.  `on_step(i, carry)` (if
    given) sees the carry *entering* step i; it must not be used together
    with autograd checkpointing.
    """
    n = len(next(iter(xs.values())))

    def scan_fn(carry, i0, i1):
        outs = []
        for i in range(i0, i1):
            if on_step is not None:
                on_step(i, carry)
            carry, y = f(carry, {k: v[i] for k, v in xs.items()})
            outs.append(y)
        return carry, torch.stack(outs)

    if checkpoint_group > 0:
        outs = []
        carry = init
        for k in range(0, n, checkpoint_group):
            carry, sub = torch.utils.checkpoint.checkpoint(
                scan_fn, carry, k, min(k + checkpoint_group, n), use_reentrant=False)
            outs.append(sub)
        return carry, torch.cat(outs, dim=0)
    return scan_fn(init, 0, n)


def _permute_in(xs):
    return {k: v.permute(2, 0, 1, 3, 4) for k, v in xs.items()}


def ttt_linear(XK, XQ, XV, eta, ttt_norm_weight, ttt_norm_bias, W1_init, b1_init,
               checkpoint_group_size, eps: float = LN_EPS, return_state: bool = False, mini_batch=None):
    """ops/ttt_linear.py:57-84.  Returns [B,NC,K,H,F] (and the final state if asked).
    `mini_batch` replaces linear_mini_batch (e.g. by its torch.compile'd form,
    as ops/ttt_linear.py:8 compiles its own)."""
    init = {"W1_states": W1_init, "b1_states": b1_init,
            "ttt_norm_weight": ttt_norm_weight, "ttt_norm_bias": ttt_norm_bias}
    xs = _permute_in({"XK": XK, "XQ": XQ, "XV": XV, "eta": eta})
    f = mini_batch or linear_mini_batch
    step = lambda p, x: f(p, x, eps)  # noqa: E731
    carry, out = scan(step, init, xs, checkpoint_group_size)
    out = out.permute(1, 0, 3, 2, 4)
    return (out, carry) if return_state else out


def ttt_mlp(XK, XQ, XV, eta, ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, W2_init, b2_init,
            checkpoint_group_size, eps: float = LN_EPS, return_state: bool = False, mini_batch=None):
    """ops/ttt_mlp.py:70-99.  Returns [B,NC,K,H,F] (and the final state if asked).
    `mini_batch` replaces mlp_mini_batch (e.g. by its torch.compile'd form, as
    ops/ttt_mlp.py:9 compiles its own)."""
    init = {"W1_states": W1_init, "b1_states": b1_init, "W2_states": W2_init, "b2_states": b2_init,
            "ttt_norm_weight": ttt_norm_weight, "ttt_norm_bias": ttt_norm_bias}
    xs = _permute_in({"XK": XK, "XQ": XQ, "XV": XV, "eta": eta})
    f = mini_batch or mlp_mini_batch
    step = lambda p, x: f(p, x, eps)  # noqa: E731
    carry, out = scan(step, init, xs, checkpoint_group_size)
    out = out.permute(1, 0, 3, 2, 4)
    return (out, carry) if return_state else out


# ----------------------------------------------------------------------------
# kernel-path side outputs (checkpoints, memo, final state)
# ----------------------------------------------------------------------------

_STATE_KEYS_LINEAR = ("W1_states", "b1_states")
_STATE_KEYS_MLP = ("W1_states", "b1_states", "W2_states", "b2_states")


def _run_states(step, init, XQ, XK, XV, eta, keys, eps):
    """Run the mini-batch recurrence without autograd, returning
    (out [B,H,NC,K,F], states entering each step [NC+1 entries, last = final])."""
    NC = XQ.shape[2]
    p = dict(init)
    states = []
    outs = []
    with torch.no_grad():
        for i in range(NC):
            states.append({k: p[k] for k in keys})
            p, y = step(p, {"XQ": XQ[:, :, i], "XK": XK[:, :, i], "XV": XV[:, :, i], "eta": eta[:, :, i]}, eps)
            outs.append(y)
        states.append({k: p[k] for k in keys})
    return torch.stack(outs, dim=2), states


def linear_forward_full(ln_w, ln_b, W1, b1, XQ, XV, XK, eta, G, eps: float = LN_EPS):
    """Everything the linear forward kernel writes, in the kernel layouts.

    Returns dict(out [B,H,NC,K,F], W1_last, b1_last, W1_ckpt [B,H,ceil(NC/G),F,F],
    b1_ckpt [B,H,ceil(NC/G),1,F]).  Checkpoint k = state entering step k*G.
    """
    init = {"W1_states": W1, "b1_states": b1, "ttt_norm_weight": ln_w, "ttt_norm_bias": ln_b}
    out, states = _run_states(linear_mini_batch, init, XQ, XK, XV, eta, _STATE_KEYS_LINEAR, eps)
    NC = XQ.shape[2]
    ks = list(range(0, NC, G))
    return {
        "out": out,
        "W1_last": states[-1]["W1_states"], "b1_last": states[-1]["b1_states"],
        "W1_ckpt": torch.stack([states[k]["W1_states"] for k in ks], dim=2),
        "b1_ckpt": torch.stack([states[k]["b1_states"] for k in ks], dim=2),
    }


def mlp_forward_full(ln_w, ln_b, W1, b1, W2, b2, XQ, XV, XK, eta, G, M: int = 0, eps: float = LN_EPS):
    """Everything the MLP forward kernel writes (out, *_last, *_ckpt, and
    *_memo when M > 0: memo s = state after mini-batch s*M is applied)."""
    init = {"W1_states": W1, "b1_states": b1, "W2_states": W2, "b2_states": b2,
            "ttt_norm_weight": ln_w, "ttt_norm_bias": ln_b}
    out, states = _run_states(mlp_mini_batch, init, XQ, XK, XV, eta, _STATE_KEYS_MLP, eps)
    NC = XQ.shape[2]
    ks = list(range(0, NC, G))
    res = {"out": out}
    for key, name in zip(_STATE_KEYS_MLP, ("W1", "b1", "W2", "b2")):
        res[name + "_last"] = states[-1][key]
        res[name + "_ckpt"] = torch.stack([states[k][key] for k in ks], dim=2)
        if M > 0:
            res[name + "_memo"] = torch.stack([states[s + 1][key] for s in range(0, NC, M)], dim=2)
    return res


def cached_readout(XQ_seg, W1, b1, W2, b2, ln_w, ln_b, eps: float = 1e-6, dtype=torch.float32):
    """Fixed-weight MLP readout XQ + LN(gelu(XQ W1 + b1) W2 + b2), with the
    per-(b,h) weights the reference kernel meant to use.
    kernels/mlp_cached_readout.py:88-109,143 (eps 1e-6 there).

    XQ_seg [B,H,S,K,F]; W1 [B,H,F,FF]; b1 [B,H,1,FF]; W2 [B,H,FF,F]; b2 [B,H,1,F]; ln [H,F].
    Returns XQ_seg + readout, in float32 (the reference's type promotion) unless
    `dtype` asks for another compute type.
    """
    H, Fd = XQ_seg.shape[1], XQ_seg.shape[-1]
    x = XQ_seg.to(dtype)
    Z1 = x @ W1.to(dtype)[:, :, None] + b1.to(dtype)[:, :, None]
    Z2 = gelu_tanh(Z1) @ W2.to(dtype)[:, :, None] + b2.to(dtype)[:, :, None]
    g = ln_w.to(dtype).reshape(1, H, 1, 1, Fd)
    bt = ln_b.to(dtype).reshape(1, H, 1, 1, Fd)
    return x + ln_fwd(Z2, g, bt, eps)


def memo_combine(XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, M: int,
                 eps: float = 1e-6, dtype=torch.float64):
    """The TTT-MLP memory-cache combiner of TTTMLP.ttt, ttt_layer.py:506-561.

    The sequence is cut into segments of M mini-batches.  Segment 0 keeps its
    output.  For a token t of segment i >= 1, with summary_j = mean of XK over
    segment j, sims_j = XU_t . summary_j for j = 0..i and gamma = softmax(sims):
        out_t = gamma_i XQW_t + sum_{j<i} gamma_j R_j(XQ_t)
    where R_j is the cached readout with the memo state j (no gradient).
    Gradients flow into XQW, XU and XK, as in the reference: the current
    segment's summary enters its own sims without detach (ttt_layer.py:519,528)
    and is cached detached (:521,559), so XK of segment i gets a gradient only
    through segment i's current-summary term.

    XQ, XK, XU, XQW [B,H,NC,K,F]; *_memo [B,H,NS,...] with NS = ceil(NC/M);
    ln_w, ln_b [H,F].  Computes in `dtype` (the reference's bf16 casts of gamma
    and of the cached sum are not reproduced).  Returns [B,H,NC,K,F].
    """
    NC = XQ.shape[2]
    NS = ceil_div(NC, M)
    outs, summaries = [], []
    for i in range(NS):
        s0, s1 = i * M, min((i + 1) * M, NC)
        xq = XQ[:, :, s0:s1].to(dtype)
        xu = XU[:, :, s0:s1].to(dtype)
        xqw = XQW[:, :, s0:s1].to(dtype)
        summ = XK[:, :, s0:s1].to(dtype).mean(dim=(2, 3))  # [B,H,F]
        if i == 0:
            summaries.append(summ.detach())
            outs.append(xqw)
            continue
        sims = torch.stack([(xu * sm[:, :, None, None, :]).sum(-1) for sm in summaries + [summ]], dim=-1)
        gam = torch.softmax(sims, dim=-1)  # [B,H,nc,K,i+1]
        acc = gam[..., i:i + 1] * xqw
        for j in range(i):
            with torch.no_grad():
                r = cached_readout(xq, W1_memo[:, :, j], b1_memo[:, :, j], W2_memo[:, :, j], b2_memo[:, :, j],
                                   ln_w, ln_b, eps, dtype=dtype)
            acc = acc + gam[..., j:j + 1] * r
        outs.append(acc)
        summaries.append(summ.detach())
    return torch.cat(outs, dim=2)


# ----------------------------------------------------------------------------
# synthetic inputs (seeded; shapes and distributions of the benchmark configs)
# ----------------------------------------------------------------------------

def eta_from_lr(lr: torch.Tensor, kind: str = "causal") -> torch.Tensor:
    """Expand per-token learning rates lr [B,H,NC,K] into a [B,H,NC,K,K] eta.

    kind="causal": eta[i,j] = lr[j]/(i+1) for j <= i, else 0.
    kind="layer":  eta[i,j] = lr[j]/K for every i (ttt_layer.py:306-309: the
                   layer multiplies the repeated get_eta output by 1/K).
    kind="tokens": eta[i,j] = lr[j] for every i.
    """
    K = lr.shape[-1]
    if kind == "layer":
        return (lr / K)[..., None, :].expand(*lr.shape[:-1], K, K).contiguous()
    if kind == "tokens":
        return lr[..., None, :].expand(*lr.shape[:-1], K, K).contiguous()
    if kind == "causal":
        i = torch.arange(K, dtype=lr.dtype)
        scale = torch.tril(torch.ones(K, K, dtype=lr.dtype)) / (i + 1)[:, None]
        return lr[..., None, :] * scale
    raise ValueError(kind)


def make_eta(u: torch.Tensor, F_: int, kind: str = "causal") -> torch.Tensor:
    """Build a [B,H,NC,K,K] eta from u [B,H,NC,K]: lr = sigmoid(u)/F, then
    eta_from_lr(lr, kind)."""
    return eta_from_lr(torch.sigmoid(u) / F_, kind)


def make_inputs(B, H, NC, K, F_, FF: int = 0, seed: int = 0, dtype=torch.float32,
                eta_kind: str = "causal", with_grad: bool = False):
    """Seeded synthetic inputs: one CPU generator, drawn in the order XQ, XK,
    XV ~ N(0,1) [B,H,NC,K,F]; u ~ N(0,1) [B,H,NC,K]; W1 ~ N(0,0.02) [H,F,F or FF];
    W2 ~ N(0,0.02) [H,FF,F] (MLP only); dOut ~ N(0,1) (if with_grad).
    Biases 0, LN weight 1 / bias 0; W tiled over B.  Activations are drawn in
    fp32 and rounded to `dtype`; state stays fp32.
    """
    gen = torch.Generator().manual_seed(seed)
    shp = (B, H, NC, K, F_)
    XQ = torch.randn(shp, generator=gen)
    XK = torch.randn(shp, generator=gen)
    XV = torch.randn(shp, generator=gen)
    u = torch.randn((B, H, NC, K), generator=gen)
    hid = FF if FF else F_
    W1 = torch.randn((H, F_, hid), generator=gen) * 0.02
    d = {}
    if FF:
        W2 = torch.randn((H, FF, F_), generator=gen) * 0.02
        d["W2"] = W2[None].repeat(B, 1, 1, 1).contiguous()
        d["b2"] = torch.zeros(B, H, 1, F_)
    if with_grad:
        d["dOut"] = torch.randn(shp, generator=gen).to(dtype)
    eta = make_eta(u, F_, eta_kind)
    d.update({
        "XQ": XQ.to(dtype), "XK": XK.to(dtype), "XV": XV.to(dtype), "eta": eta.to(dtype),
        "W1": W1[None].repeat(B, 1, 1, 1).contiguous(),
        "b1": torch.zeros(B, H, 1, hid),
        "ln_w": torch.ones(H, F_), "ln_b": torch.zeros(H, F_),
    })
    return d


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def linear_flops_per_token_head(K: int, F_: int) -> int:
    """Dual-form forward FLOPs per token-head: 6F^2 + 6KF."""
    return 6 * F_ * F_ + 6 * K * F_


def mlp_flops_per_token_head(K: int, F_: int, FF: int) -> int:
    """Dual-form forward FLOPs per token-head: 14*F*FF + 6K*FF + 6K*F."""
    return 14 * F_ * FF + 6 * K * FF + 6 * K * F_

