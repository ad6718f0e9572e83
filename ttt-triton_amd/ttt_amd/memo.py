"""TTT-MLP memory-cache combiner on the HIP path: the segment loop of
`TTTMLP.ttt` (ttt_layer.py:506-561) as two fused launches per direction
instead of one cached-readout launch per (segment, memo state) pair.

For a token of segment i >= 1 (segments of M mini-batches), with
summary_j = mean of XK over segment j and gamma = softmax_j(XU . summary_j)
over j = 0..i:

    out = gamma_i XQW + sum_{j<i} gamma_j (XQ + LN_1e-6(gelu(XQ W1_j + b1_j) W2_j + b2_j) ln_w + ln_b)

Segment 0 keeps XQW.  The memo states are the `TritonMLP.apply` memo outputs
with the same M.  Gradients flow into XQW, XU and XK, as in the reference: it
runs the cached readouts under `torch.no_grad`, and a segment's summary enters
its own tokens' gates undetached (ttt_layer.py:519,528) but is cached detached
(:521,559), so XK of a segment gets the mean-summary gradient of its own
segment only.  Unlike the reference's cached-readout kernel, every (b,h)
chain uses its own memo states.

Layouts follow the caller (ttt_layer.py:453-561): XQ, XK, XU, XQW
[B,H,NC,K,F]; W1_memo [B,H,NS,F,FF], b1_memo [B,H,NS,1,FF], W2_memo
[B,H,NS,FF,F], b2_memo [B,H,NS,1,F] fp32; LN parameters [H,F]."""

from __future__ import annotations

import math

import torch

from . import _lib
from ._common import as_act, check_device, dtype_code, ptr, stream_of

READOUT_EPS = 1e-6  # kernels/mlp_cached_readout.py:98


def _check(XQ, XK, XU, XQW, W1, b1, W2, b2, ln_w, ln_b, M):
    if XQ.dim() != 5:
        raise ValueError(f"XQ must be [B,H,NC,K,F], got {tuple(XQ.shape)}")
    B, H, NC, K, F = XQ.shape
    for name, t in (("XK", XK), ("XU", XU), ("XQW", XQW)):
        if tuple(t.shape) != (B, H, NC, K, F):
            raise ValueError(f"{name} shape {tuple(t.shape)} != XQ shape {tuple(XQ.shape)}")
    M = int(M)
    if M < 1:
        raise ValueError(f"memo segment size M must be >= 1, got {M}")
    NS = math.ceil(NC / M)
    FF = W1.shape[-1]
    want = {"W1_memo": (W1, (B, H, NS, F, FF)), "b1_memo": (b1, (B, H, NS, 1, FF)),
            "W2_memo": (W2, (B, H, NS, FF, F)), "b2_memo": (b2, (B, H, NS, 1, F))}
    for name, (t, shp) in want.items():
        if tuple(t.shape) != shp:
            raise ValueError(f"{name} must be {shp}, got {tuple(t.shape)}")
    if tuple(ln_w.shape) != (H, F) or tuple(ln_b.shape) != (H, F):
        raise ValueError(f"LN weight/bias must be [H,F]={(H, F)}")
    return B, H, NC, K, F, FF, M


def _f32(t):
    return t.detach().to(torch.float32).contiguous()


def memo_combine_forward(XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, M: int,
                         eps: float = READOUT_EPS, images: bool = True):
    """Run the combiner.  Returns (out [B,H,NC,K,F] in XQW.dtype, gates) where
    `gates` (uint8 device buffer) is what memo_combine_backward needs.  With
    `images` (bf16), the workspace also holds each memo state's LDS image,
    written once here and copied straight into LDS by this call and the
    backward: worth its one conversion pass when a backward follows; without
    it every workgroup converts the states it stages (the same results)."""
    B, H, NC, K, F, FF, M = _check(XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, M)
    dev = check_device(XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b)
    mp = XQW.dtype
    code = dtype_code(mp)
    xq, xk, xu, xqw = (as_act(t, mp) for t in (XQ, XK, XU, XQW))
    ws = [_f32(t) for t in (W1_memo, b1_memo, W2_memo, b2_memo)]
    lw, lb = _f32(ln_w), _f32(ln_b)
    lib = _lib.load()
    # the gates and, for bf16, the memo states' LDS images that both calls copy in
    nbytes = (lib.ttt_mlp_memo_workspace_bytes(B, H, NC, K, F, FF, M, code) if images
              else lib.ttt_mlp_memo_gates_bytes(B, H, NC, K, F, M))
    gates = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    out = torch.empty((B, H, NC, K, F), device=dev, dtype=mp)
    with torch.cuda.device(dev):
        st = lib.ttt_mlp_memo_combine(ptr(xq), ptr(xk), ptr(xu), ptr(xqw), *(ptr(t) for t in ws), ptr(lw), ptr(lb),
                                      B, H, NC, K, F, FF, M, code, float(eps), ptr(out), ptr(gates), gates.numel(),
                                      stream_of(dev))
    _lib.check(st, "ttt_mlp_memo_combine")
    return out, gates


def memo_combine_backward(XQ, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, M: int, gates, dout,
                          eps: float = READOUT_EPS):
    """Gradients (dXK, dXU, dXQW) in XQW.dtype of the combiner run that produced `gates`."""
    B, H, NC, K, F = XQ.shape
    FF = W1_memo.shape[-1]
    dev = check_device(XQ, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, gates, dout)
    mp = XQW.dtype
    code = dtype_code(mp)
    xq, xu, xqw, do = (as_act(t, mp) for t in (XQ, XU, XQW, dout))
    ws = [_f32(t) for t in (W1_memo, b1_memo, W2_memo, b2_memo)]
    lw, lb = _f32(ln_w), _f32(ln_b)
    dxk, dxu, dxqw = (torch.empty((B, H, NC, K, F), device=dev, dtype=mp) for _ in range(3))
    lib = _lib.load()
    with torch.cuda.device(dev):
        st = lib.ttt_mlp_memo_combine_bwd(ptr(xq), ptr(xu), ptr(xqw), *(ptr(t) for t in ws), ptr(lw), ptr(lb),
                                          ptr(do), B, H, NC, K, F, FF, int(M), code, float(eps), ptr(gates),
                                          gates.numel(), ptr(dxk), ptr(dxu), ptr(dxqw), stream_of(dev))
    _lib.check(st, "ttt_mlp_memo_combine_bwd")
    return dxk, dxu, dxqw


class MemoCombineFunction(torch.autograd.Function):
    """apply(XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, M[, eps]) -> out.
    Differentiable wrt XK, XU and XQW (as the reference's loop is)."""

    @staticmethod
    def forward(ctx, XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, M, eps=READOUT_EPS):
        # the memo-state images pay off only when the backward runs too
        training = any(ctx.needs_input_grad[1:4])
        out, gates = memo_combine_forward(XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, M, eps,
                                          images=training)
        ctx.save_for_backward(XQ, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, gates)
        ctx.M, ctx.eps = int(M), eps
        ctx.dtypes = (XK.dtype, XU.dtype, XQW.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        XQ, XU, XQW, W1, b1, W2, b2, lw, lb, gates = ctx.saved_tensors
        dxk, dxu, dxqw = memo_combine_backward(XQ, XU, XQW, W1, b1, W2, b2, lw, lb, ctx.M, gates, dout, ctx.eps)
        return (None, dxk.to(ctx.dtypes[0]), dxu.to(ctx.dtypes[1]), dxqw.to(ctx.dtypes[2])) + (None,) * 8


def mlp_memo_combine(XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, M: int):
    """Drop-in for the segment loop of TTTMLP.ttt (ttt_layer.py:506-561): given
    the TritonMLP.apply output XQW_batch and memo, returns the combined
    XQW_batch [B,H,NC,K,F] (before the caller's permute/reshape)."""
    return MemoCombineFunction.apply(XQ, XK, XU, XQW, W1_memo, b1_memo, W2_memo, b2_memo, ln_w, ln_b, int(M))


__all__ = ["mlp_memo_combine", "MemoCombineFunction", "memo_combine_forward", "memo_combine_backward"]
