"""TTT-Linear on the HIP path: forward/backward launchers and the autograd
Function behind `linear_triton.TritonLinear` and `ops.ttt_linear`.

Semantics are the reference ops path's (ops/ttt_linear.py:8-84): dual form
with a general KxK eta, LayerNorm eps 1e-8, gradient of every input including
a dense eta gradient.  Layouts follow TritonLinear (linear_triton.py:62-265):
activations [B,H,NC,K,F], eta [B,H,NC,K,K], fast weights [B,H,F,F] and
[B,H,1,F], LN parameters [H,F]."""

from __future__ import annotations

import math

import torch

from . import _lib
from ._common import as_act, check_device, dtype_code, eta_operand, ptr, stream_of

LN_EPS = 1e-8  # ops/ttt_utils.py:4,21


def _check_shapes(ln_w, ln_b, W1, b1, XQ, XV, XK, eta, rule=_lib.ETA_DENSE):
    if XQ.dim() != 5:
        raise ValueError(f"XQ must be [B,H,NC,K,F], got {tuple(XQ.shape)}")
    B, H, NC, K, F = XQ.shape
    for name, t in (("XK", XK), ("XV", XV)):
        if tuple(t.shape) != (B, H, NC, K, F):
            raise ValueError(f"{name} shape {tuple(t.shape)} != XQ shape {tuple(XQ.shape)}")
    if rule == _lib.ETA_DENSE and tuple(eta.shape) != (B, H, NC, K, K):
        raise ValueError(f"eta must be [B,H,NC,K,K]={(B, H, NC, K, K)}, got {tuple(eta.shape)}")
    if rule != _lib.ETA_DENSE and tuple(eta.shape) != (B, H, NC, K):
        raise ValueError(f"lr must be [B,H,NC,K]={(B, H, NC, K)}, got {tuple(eta.shape)}")
    if tuple(W1.shape) != (B, H, F, F):
        raise ValueError(f"W1 must be [B,H,F,F]={(B, H, F, F)}, got {tuple(W1.shape)}")
    if tuple(b1.shape) != (B, H, 1, F):
        raise ValueError(f"b1 must be [B,H,1,F]={(B, H, 1, F)}, got {tuple(b1.shape)}")
    if tuple(ln_w.shape) != (H, F) or tuple(ln_b.shape) != (H, F):
        raise ValueError(f"LN weight/bias must be [H,F]={(H, F)}")
    return B, H, NC, K, F


def linear_forward(ln_w, ln_b, W1, b1, XQ, XV, XK, eta, G: int, eps: float = LN_EPS,
                   want_ckpt: bool = True, want_last: bool = False, want_saved: bool = False,
                   eta_rule="dense"):
    """Run the forward kernel.  `eta` is the dense [B,H,NC,K,K] tensor
    (eta_rule "dense") or the learning rates lr [B,H,NC,K] expanded on chip
    by eta_rule "layer" or "causal".  Returns (out [B,H,NC,K,F] in XQ.dtype,
    (W1_ckpt, b1_ckpt) or None, (W1_last, b1_last) or None, saved or None).

    `saved` (uint8, ttt_linear_saved_bytes long) holds what linear_backward
    reads instead of re-running the forward; the backward needs it together
    with W1_ckpt and W1_last."""
    rule = _lib.eta_rule_code(eta_rule)
    B, H, NC, K, F = _check_shapes(ln_w, ln_b, W1, b1, XQ, XV, XK, eta, rule)
    dev = check_device(XQ, XK, XV, eta, W1, b1, ln_w, ln_b)
    mp = XQ.dtype
    code = dtype_code(mp)
    G = int(G)
    NK = math.ceil(NC / G)
    xq, xk, xv = (as_act(t, mp) for t in (XQ, XK, XV))
    et, krule = eta_operand(eta, rule, mp)
    w1 = W1.detach().to(torch.float32).contiguous()
    bb = b1.detach().to(torch.float32).contiguous()
    lw = ln_w.detach().to(torch.float32).contiguous()
    lb = ln_b.detach().to(torch.float32).contiguous()
    out = torch.empty((B, H, NC, K, F), device=dev, dtype=mp)
    ck = last = None
    if want_ckpt:
        ck = (torch.empty((B, H, NK, F, F), device=dev, dtype=torch.float32),
              torch.empty((B, H, NK, 1, F), device=dev, dtype=torch.float32))
    if want_last:
        last = (torch.empty((B, H, F, F), device=dev, dtype=torch.float32),
                torch.empty((B, H, 1, F), device=dev, dtype=torch.float32))
    lib = _lib.load()
    saved = None
    if want_saved or not _lib.fast_linear_shape(K, F):
        nbytes = lib.ttt_linear_saved_bytes(B, H, NC, K, F)
        saved = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        st = lib.ttt_linear_fwd(
            ptr(xq), ptr(xk), ptr(xv), ptr(et), ptr(lw), ptr(lb), ptr(w1), ptr(bb),
            B, H, NC, K, F, G, code, krule, float(eps), ptr(out),
            ptr(last[0]) if last else None, ptr(last[1]) if last else None,
            ptr(ck[0]) if ck else None, ptr(ck[1]) if ck else None,
            ptr(saved) if saved is not None else None, saved.numel() if saved is not None else 0,
            stream_of(dev))
    _lib.check(st, "ttt_linear_fwd")
    return out, ck, last, saved


def linear_backward(ln_w, ln_b, XQ, XV, XK, eta, W1_ckpt, W1_last, saved, dout, G: int, eps: float = LN_EPS,
                    eta_rule="dense", sum_ln: bool = True):
    """Run the backward kernel on what linear_forward(want_ckpt, want_last,
    want_saved) returned.  Returns fp32 (dln_w [H,F], dln_b [H,F],
    dW1 [B,H,F,F], db1 [B,H,1,F]) and (dXQ, dXV, dXK, deta) in XQ.dtype,
    deta being dlr [B,H,NC,K] fp32 for an lr eta rule, and fp32 for a dense
    fp32 eta under 16-bit activations (read in fp32 too).  With sum_ln=False
    dln_w and dln_b are the per-chain partials [B,H,F]."""
    rule = _lib.eta_rule_code(eta_rule)
    B, H, NC, K, F = XQ.shape
    dev = check_device(XQ, XK, XV, eta, W1_ckpt, W1_last, saved, dout)
    mp = XQ.dtype
    code = dtype_code(mp)
    xq, xk, xv, do = (as_act(t, mp) for t in (XQ, XK, XV, dout))
    et, krule = eta_operand(eta, rule, mp)
    lw = ln_w.detach().to(torch.float32).contiguous()
    lb = ln_b.detach().to(torch.float32).contiguous()
    dxq = torch.empty_like(xq)
    dxk = torch.empty_like(xq)
    dxv = torch.empty_like(xq)
    deta = torch.empty_like(et)
    dW = torch.empty((B, H, F, F), device=dev, dtype=torch.float32)
    db = torch.empty((B, H, 1, F), device=dev, dtype=torch.float32)
    dlw = torch.empty((B, H, F), device=dev, dtype=torch.float32)
    dlb = torch.empty((B, H, F), device=dev, dtype=torch.float32)
    lib = _lib.load()
    with torch.cuda.device(dev):
        st = lib.ttt_linear_bwd(
            ptr(xq), ptr(xk), ptr(xv), ptr(et), ptr(lw), ptr(lb), ptr(W1_ckpt), ptr(W1_last), ptr(do),
            B, H, NC, K, F, int(G), code, krule, float(eps),
            ptr(dxq), ptr(dxk), ptr(dxv), ptr(deta), ptr(dW), ptr(db), ptr(dlw), ptr(dlb),
            ptr(saved), saved.numel(), stream_of(dev))
    _lib.check(st, "ttt_linear_bwd")
    if sum_ln:
        dlw, dlb = dlw.sum(0), dlb.sum(0)
    return (dlw, dlb, dW, db), (dxq, dxv, dxk, deta)


class TTTLinearFunction(torch.autograd.Function):
    """autograd Function with TritonLinear's signature (linear_triton.py:15-60):
    apply(ln_w, ln_b, W1_init, b1_init, XQ, XV, XK, eta, checkpoint_group_size[, eps[, eta_rule]])
    -> XQW [B,H,NC,K,F] in XQ.dtype.  With eta_rule "layer" or "causal",
    eta is the learning-rate tensor lr [B,H,NC,K] expanded on chip."""

    @staticmethod
    def forward(ctx, ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, XQ_batch, XV_batch, XK_batch, eta_batch,
                checkpoint_group_size, eps=LN_EPS, eta_rule="dense"):
        NC = XQ_batch.shape[2]
        G = min(max(int(checkpoint_group_size), 1), NC)
        # what the backward reads only when a gradient is wanted
        train = any(ctx.needs_input_grad)
        out, ck, last, saved = linear_forward(ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, XQ_batch,
                                              XV_batch, XK_batch, eta_batch, G, eps, want_ckpt=train,
                                              want_last=train, want_saved=train, eta_rule=eta_rule)
        if train:
            ctx.save_for_backward(XQ_batch, XV_batch, XK_batch, eta_batch, ttt_norm_weight, ttt_norm_bias, ck[0],
                                  last[0], saved)
        ctx.G, ctx.eps, ctx.eta_rule = G, eps, eta_rule
        ctx.dtypes = (ttt_norm_weight.dtype, ttt_norm_bias.dtype, W1_init.dtype, b1_init.dtype,
                      XQ_batch.dtype, XV_batch.dtype, XK_batch.dtype, eta_batch.dtype)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        XQ, XV, XK, eta, lw, lb, Wc, Wl, saved = ctx.saved_tensors
        (dlw, dlb, dW, db), (dxq, dxv, dxk, deta) = linear_backward(
            lw, lb, XQ, XV, XK, eta, Wc, Wl, saved, grad_out, ctx.G, ctx.eps, eta_rule=ctx.eta_rule)
        grads = (dlw, dlb, dW, db, dxq, dxv, dxk, deta)
        grads = tuple(gr.to(dt) for gr, dt in zip(grads, ctx.dtypes))
        return grads + (None, None, None)
