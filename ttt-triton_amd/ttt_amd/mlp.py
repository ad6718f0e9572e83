"""TTT-MLP on the HIP path: forward/backward launchers, the autograd Function
behind `mlp_triton.TritonMLP` and `ops.ttt_mlp`, and the fixed-weight readout
behind `kernels.mlp_cached_readout.mlp_cached_readout_triton`.

Semantics are the reference ops path's (ops/ttt_mlp.py:9-99): two-layer
GELU(tanh) fast-weight MLP, dual form for both layers with a general KxK eta,
LayerNorm eps 1e-8, gradients of every input including a dense eta gradient.
Layouts follow TritonMLP (mlp_triton.py:71-351): W1 [B,H,F,FF], b1 [B,H,1,FF],
W2 [B,H,FF,F], b2 [B,H,1,F]; memo snapshots [B,H,NS,...] fp32."""

from __future__ import annotations

import math
import os

import torch

from . import _lib
from ._common import as_act, check_device, dtype_code, eta_operand, ptr, stream_of

LN_EPS = 1e-8  # ops/ttt_utils.py:4,21

# With TTT_AMD_CHECK=1 every backward waits for its launch and raises if a
# fused dXQ/dXK worker gave up waiting (its rows are then NaN).
CHECK_BWD = os.environ.get("TTT_AMD_CHECK", "0") not in ("", "0")


def _f32(t):
    return t.detach().to(torch.float32).contiguous()


def _check_shapes(ln_w, ln_b, W1, b1, W2, b2, XQ, XV, XK, eta, rule=_lib.ETA_DENSE):
    if XQ.dim() != 5:
        raise ValueError(f"XQ must be [B,H,NC,K,F], got {tuple(XQ.shape)}")
    B, H, NC, K, F = XQ.shape
    FF = W1.shape[-1]
    for name, t in (("XK", XK), ("XV", XV)):
        if tuple(t.shape) != (B, H, NC, K, F):
            raise ValueError(f"{name} shape {tuple(t.shape)} != XQ shape {tuple(XQ.shape)}")
    if rule == _lib.ETA_DENSE and tuple(eta.shape) != (B, H, NC, K, K):
        raise ValueError(f"eta must be [B,H,NC,K,K]={(B, H, NC, K, K)}, got {tuple(eta.shape)}")
    if rule != _lib.ETA_DENSE and tuple(eta.shape) != (B, H, NC, K):
        raise ValueError(f"lr must be [B,H,NC,K]={(B, H, NC, K)}, got {tuple(eta.shape)}")
    # mlp_triton.py:91-94
    if tuple(W1.shape) != (B, H, F, FF):
        raise ValueError(f"W1 must be [B,H,F,FF]={(B, H, F, FF)}, got {tuple(W1.shape)}")
    if tuple(b1.shape) != (B, H, 1, FF):
        raise ValueError(f"b1 must be [B,H,1,FF]={(B, H, 1, FF)}, got {tuple(b1.shape)}")
    if tuple(W2.shape) != (B, H, FF, F):
        raise ValueError(f"W2 must be [B,H,FF,F]={(B, H, FF, F)}, got {tuple(W2.shape)}")
    if tuple(b2.shape) != (B, H, 1, F):
        raise ValueError(f"b2 must be [B,H,1,F]={(B, H, 1, F)}, got {tuple(b2.shape)}")
    if tuple(ln_w.shape) != (H, F) or tuple(ln_b.shape) != (H, F):
        raise ValueError(f"LN weight/bias must be [H,F]={(H, F)}")
    return B, H, NC, K, F, FF


def mlp_forward(ln_w, ln_b, W1, b1, W2, b2, XQ, XV, XK, eta, G: int, M: int = 0, eps: float = LN_EPS,
                want_ckpt: bool = True, want_last: bool = False, want_saved: bool = False,
                ckpt_w1_only: bool = False, eta_rule="dense"):
    """Run the forward kernel.  `eta` is the dense [B,H,NC,K,K] tensor
    (eta_rule "dense") or the learning rates lr [B,H,NC,K] that the kernel
    expands by eta_rule "layer" (lr[j]/K in every row) or "causal"
    (lr[j]/(i+1) for j <= i).  Returns (out [B,H,NC,K,F] in XQ.dtype,
    ckpt (W1,b1,W2,b2) or None, memo (W1,b1,W2,b2) or None, last or None,
    saved or None).  ckpt, last and saved are what mlp_backward needs: the
    checkpoints every G mini-batches, the final state, and each mini-batch's
    state-update operands and activations (a flat uint8 buffer of
    ttt_mlp_saved_bytes).  The backward reads only W1's checkpoints: with
    ckpt_w1_only the other three are neither allocated nor written (None)."""
    rule = _lib.eta_rule_code(eta_rule)
    B, H, NC, K, F, FF = _check_shapes(ln_w, ln_b, W1, b1, W2, b2, XQ, XV, XK, eta, rule)
    dev = check_device(XQ, XK, XV, eta, W1, b1, W2, b2, ln_w, ln_b)
    mp = XQ.dtype
    code = dtype_code(mp)
    G = int(G)
    NK = math.ceil(NC / G)
    xq, xk, xv = (as_act(t, mp) for t in (XQ, XK, XV))
    et, krule = eta_operand(eta, rule, mp)
    w1, bb1, w2, bb2, lw, lb = (_f32(t) for t in (W1, b1, W2, b2, ln_w, ln_b))
    out = torch.empty((B, H, NC, K, F), device=dev, dtype=mp)

    def state(n):
        lead = (B, H) if n is None else (B, H, n)
        return (torch.empty(lead + (F, FF), device=dev, dtype=torch.float32),
                torch.empty(lead + (1, FF), device=dev, dtype=torch.float32),
                torch.empty(lead + (FF, F), device=dev, dtype=torch.float32),
                torch.empty(lead + (1, F), device=dev, dtype=torch.float32))

    ck = state(NK) if want_ckpt else None
    if ck is not None and ckpt_w1_only:
        ck = (ck[0], None, None, None)
    memo = state(math.ceil(NC / M)) if M and M > 0 else None
    last = state(None) if want_last else None
    none4 = (None, None, None, None)
    lib = _lib.load()
    saved = None
    if want_saved or not _lib.fast_mlp_shape(K, F, FF):
        saved = torch.empty(lib.ttt_mlp_saved_bytes(B, H, NC, K, F, FF, code), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        st = lib.ttt_mlp_fwd(
            ptr(xq), ptr(xk), ptr(xv), ptr(et), ptr(lw), ptr(lb), ptr(w1), ptr(bb1), ptr(w2), ptr(bb2),
            B, H, NC, K, F, FF, G, int(M) if M else 0, code, krule, float(eps), ptr(out),
            *(tuple(ptr(t) for t in last) if last else none4),
            *(tuple(ptr(t) if t is not None else None for t in ck) if ck else none4),
            *(tuple(ptr(t) for t in memo) if memo else none4),
            ptr(saved) if saved is not None else None, saved.numel() if saved is not None else 0,
            stream_of(dev))
    _lib.check(st, "ttt_mlp_fwd")
    return out, ck, memo, last, saved


def mlp_backward(ln_w, ln_b, XQ, XV, XK, eta, ckpt, last, saved, dout, G: int, eps: float = LN_EPS,
                 workspace=None, eta_rule="dense", check_timeout=None, sum_ln: bool = True):
    """Run the backward kernel.  ckpt = (W1, b1, W2, b2) checkpoints, last =
    the final state and saved = the saved buffer, all from one mlp_forward
    call with the same G and eta form.  `workspace` (uint8, at least
    ttt_mlp_bwd_workspace_bytes) is allocated here when not given; for the
    register-resident shapes (F = FF = 32) one of at least 256 bytes runs
    their one-launch backward instead of the two-launch one.  Returns
    fp32 (dln_w [H,F], dln_b [H,F], dW1, db1, dW2, db2) and (dXQ, dXV, dXK,
    deta) in XQ.dtype, deta being dlr [B,H,NC,K] fp32 for an lr eta rule, and
    fp32 for a dense fp32 eta under 16-bit activations (read in fp32 too).
    With check_timeout (default: TTT_AMD_CHECK set) the call waits for the
    launch and raises TTTError if a fused dXQ/dXK worker gave up waiting.
    With sum_ln=False dln_w and dln_b are the per-chain partials [B,H,F]."""
    rule = _lib.eta_rule_code(eta_rule)
    B, H, NC, K, F = XQ.shape
    FF = ckpt[0].shape[-1]
    dev = check_device(XQ, XK, XV, eta, dout, *(t for t in ckpt if t is not None), *last, saved)
    mp = XQ.dtype
    code = dtype_code(mp)
    xq, xk, xv, do = (as_act(t, mp) for t in (XQ, XK, XV, dout))
    et, krule = eta_operand(eta, rule, mp)
    lw, lb = _f32(ln_w), _f32(ln_b)
    dxq, dxk, dxv = torch.empty_like(xq), torch.empty_like(xq), torch.empty_like(xq)
    deta = torch.empty_like(et)
    f32 = dict(device=dev, dtype=torch.float32)
    dW1, db1 = torch.empty((B, H, F, FF), **f32), torch.empty((B, H, 1, FF), **f32)
    dW2, db2 = torch.empty((B, H, FF, F), **f32), torch.empty((B, H, 1, F), **f32)
    dlw, dlb = torch.empty((B, H, F), **f32), torch.empty((B, H, F), **f32)
    lib = _lib.load()
    nws = lib.ttt_mlp_bwd_workspace_bytes(B, H, NC, K, F, FF, code)
    ws = torch.empty(nws, device=dev, dtype=torch.uint8) if workspace is None else workspace
    with torch.cuda.device(dev):
        st = lib.ttt_mlp_bwd(
            ptr(xq), ptr(xk), ptr(xv), ptr(et), ptr(lw), ptr(lb),
            *(ptr(t) if t is not None else None for t in ckpt),
            *(ptr(t) for t in last), ptr(do),
            B, H, NC, K, F, FF, int(G), code, krule, float(eps),
            ptr(dxq), ptr(dxk), ptr(dxv), ptr(deta), ptr(dW1), ptr(db1), ptr(dW2), ptr(db2), ptr(dlw), ptr(dlb),
            ptr(saved), saved.numel(), ptr(ws), ws.numel(), stream_of(dev))
    _lib.check(st, "ttt_mlp_bwd")
    if CHECK_BWD if check_timeout is None else check_timeout:
        _lib.check(mlp_bwd_status(ws, B, H, NC, K, F, FF, code), "ttt_mlp_bwd")
    if sum_ln:
        dlw, dlb = dlw.sum(0), dlb.sum(0)
    return (dlw, dlb, dW1, db1, dW2, db2), (dxq, dxv, dxk, deta)


def mlp_bwd_status(workspace, B, H, NC, K, F, FF, code) -> int:
    """ttt_mlp_bwd_check on the workspace of the last backward that used it
    (waits for the current stream): 0, or the timeout status."""
    dev = workspace.device
    with torch.cuda.device(dev):
        return _lib.load().ttt_mlp_bwd_check(ptr(workspace), workspace.numel(), B, H, NC, K, F, FF, code,
                                             stream_of(dev))


class TTTMLPFunction(torch.autograd.Function):
    """autograd Function with TritonMLP's signature (mlp_triton.py:15-69):
    apply(ln_w, ln_b, W1, b1, W2, b2, XQ, XV, XK, eta, checkpoint_group_size,
    memo_segment_size[, eps]) -> (XQW [B,H,NC,K,F] in XQ.dtype, W1_memo, b1_memo,
    W2_memo, b2_memo); the memo snapshots are fp32 and non-differentiable.
    An optional last argument `eta_rule` ("layer" or "causal") makes eta_batch
    the learning rates lr [B,H,NC,K] expanded on chip (its gradient is dlr)."""

    @staticmethod
    def forward(ctx, ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, W2_init, b2_init, XQ_batch, XV_batch,
                XK_batch, eta_batch, checkpoint_group_size, memo_segment_size, eps=LN_EPS, eta_rule="dense"):
        NC = XQ_batch.shape[2]
        G = min(max(int(checkpoint_group_size), 1), NC)
        M = int(memo_segment_size)
        # what the backward reads (checkpoints, final state, saved buffer) only
        # when a gradient is wanted: an inference forward skips those stores
        train = any(ctx.needs_input_grad)
        out, ck, memo, last, saved = mlp_forward(ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, W2_init, b2_init,
                                               XQ_batch, XV_batch, XK_batch, eta_batch, G, M=M, eps=eps,
                                               want_ckpt=train, want_last=train, want_saved=train,
                                               ckpt_w1_only=True, eta_rule=eta_rule)
        if train:
            ctx.save_for_backward(XQ_batch, XV_batch, XK_batch, eta_batch, ttt_norm_weight, ttt_norm_bias, *ck,
                                  *last, saved)
        ctx.G, ctx.eps, ctx.eta_rule = G, eps, eta_rule
        ctx.dtypes = (ttt_norm_weight.dtype, ttt_norm_bias.dtype, W1_init.dtype, b1_init.dtype, W2_init.dtype,
                      b2_init.dtype, XQ_batch.dtype, XV_batch.dtype, XK_batch.dtype, eta_batch.dtype)
        if memo is None:
            memo = tuple(torch.empty(0, device=XQ_batch.device) for _ in range(4))
        ctx.mark_non_differentiable(*memo)
        return (out,) + tuple(memo)

    @staticmethod
    def backward(ctx, grad_out, *unused):
        XQ, XV, XK, eta, lw, lb = ctx.saved_tensors[:6]
        ck, last, saved = ctx.saved_tensors[6:10], ctx.saved_tensors[10:14], ctx.saved_tensors[14]
        (dlw, dlb, dW1, db1, dW2, db2), (dxq, dxv, dxk, deta) = mlp_backward(
            lw, lb, XQ, XV, XK, eta, ck, last, saved, grad_out, ctx.G, ctx.eps, eta_rule=ctx.eta_rule)
        grads = (dlw, dlb, dW1, db1, dW2, db2, dxq, dxv, dxk, deta)
        grads = tuple(gr.to(dt) for gr, dt in zip(grads, ctx.dtypes))
        return grads + (None, None, None, None)


READOUT_EPS = 1e-6  # kernels/mlp_cached_readout.py:98


def _states_per_chain(t: torch.Tensor, B: int, H: int, inner: int):
    """S such that `t` ([B,H,*,*]) is slice j of a contiguous [B,H,S,*,*] tensor,
    i.e. its chain stride is S*inner with contiguous inner dims; None otherwise."""
    st = t.stride()
    if st[3] != 1 or st[2] != t.shape[3] or st[1] % inner != 0:
        return None
    S = st[1] // inner
    if S < 1 or (B > 1 and st[0] != H * st[1]):
        return None
    return S


def mlp_cached_readout(XQ_seg, W1, b1, W2, b2, ln_w, ln_b, eps: float = READOUT_EPS):
    """XQ_seg + LN_eps(gelu(XQ_seg W1 + b1) W2 + b2) per (b,h) chain, fp32.

    XQ_seg [B,H,NS,K,F] (fp32 or bf16); W1 [B,H,F,FF], b1 [B,H,1,FF],
    W2 [B,H,FF,F], b2 [B,H,1,F] fp32, either contiguous or the same slice j of
    [B,H,S,...] memo tensors (read in place); ln_w, ln_b [H,F]."""
    if XQ_seg.dim() != 5:
        raise ValueError(f"XQ_seg must be [B,H,NS,K,F], got {tuple(XQ_seg.shape)}")
    B, H, NS, K, F = XQ_seg.shape
    FF = W1.shape[-1]
    want = {"W1": (W1, (B, H, F, FF)), "b1": (b1, (B, H, 1, FF)), "W2": (W2, (B, H, FF, F)),
            "b2": (b2, (B, H, 1, F))}
    for name, (t, shp) in want.items():
        if tuple(t.shape) != shp:
            raise ValueError(f"{name} must be {shp}, got {tuple(t.shape)}")
    if tuple(ln_w.shape) != (H, F) or tuple(ln_b.shape) != (H, F):
        raise ValueError(f"LN weight/bias must be [H,F]={(H, F)}")
    dev = check_device(XQ_seg, W1, b1, W2, b2, ln_w, ln_b)
    mp = XQ_seg.dtype
    code = dtype_code(mp)
    xq = as_act(XQ_seg, mp)
    ws = [W1, b1, W2, b2]
    S = None
    if all(t.dtype == torch.float32 for t in ws):
        Ss = {_states_per_chain(t, B, H, t.shape[2] * t.shape[3]) for t in ws}
        if len(Ss) == 1:
            S = Ss.pop()
    if S is None:
        ws, S = [_f32(t) for t in ws], 1
    lw, lb = _f32(ln_w), _f32(ln_b)
    out = torch.empty((B, H, NS, K, F), device=dev, dtype=torch.float32)
    lib = _lib.load()
    with torch.cuda.device(dev):
        st = lib.ttt_mlp_cached_readout(ptr(xq), *(ptr(t) for t in ws), ptr(lw), ptr(lb),
                                        B, H, NS, K, F, FF, int(S), code, float(eps), ptr(out), stream_of(dev))
    _lib.check(st, "ttt_mlp_cached_readout")
    return out
