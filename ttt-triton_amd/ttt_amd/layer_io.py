"""The producer and consumer around the inner loop on the HIP path
(ttt_qkvu_producer_* and ttt_post_norm_* in include/ttt_amd.h).

ProducerFunction: from the fused projection rows [B, L, 4*D + H (+pad)]
  (XQ | XK | XV | XU | lr logits) to the inner loop's inputs XQ, XK, XV (the
  reconstruction target), XU in [B,H,NC,K,F] and lr [B,H,NC,K] fp32:
  TTTBase.process_input after its projections (ttt_layer.py:271-309).
PostNormFunction: from the inner loop's [B,H,NC,K,F] output to post_norm's
  output [B, L, D] (ttt_layer.py:349, 563-564).
rope_table: the cos/sin table of the layer's 3-D rotary embedding
  (utils.py:24-68 for the angles, applied as utils.py:97-123 does)."""

from __future__ import annotations

import torch

from . import _lib
from ._common import check_device, dtype_code, ptr, stream_of

RECON_EPS = 1e-8     # ttt_layer.py:230
POST_NORM_EPS = 1e-6  # ttt_layer.py:78


def rope_table(head_dim: int, frames: int, height: int = 1, width: int = 1, theta: float = 10000.0) -> torch.Tensor:
    """[frames*height*width, head_dim/2, 2] fp32 (cos, sin) of the rotary
    angles for each token position (t, h, w) flattened t-major and each
    feature pair p.  The head dim is split as precompute_freqs_cis_3d splits
    it (utils.py:24-68): the first head_dim/8 pairs rotate with the frame
    index, the next 3*head_dim/16 with the row, the last 3*head_dim/16 with
    the column, each with frequencies theta^(-2i/d) over its own share d.
    Angles and their cos/sin are formed in fp32."""
    if head_dim % 16:
        raise ValueError(f"head_dim must be a multiple of 16, got {head_dim}")

    def inv_freq(d):
        return 1.0 / (theta ** (torch.arange(0, d, 2)[: d // 2].float() / d))

    dt, dh = head_dim // 4, head_dim // 8 * 3
    ang_t = torch.arange(frames, dtype=torch.float32)[:, None] * inv_freq(dt)[None, :]
    ang_h = torch.arange(height, dtype=torch.float32)[:, None] * inv_freq(dh)[None, :]
    ang_w = torch.arange(width, dtype=torch.float32)[:, None] * inv_freq(dh)[None, :]
    n_t, n_h, n_w = ang_t.shape[1], ang_h.shape[1], ang_w.shape[1]
    ang = torch.cat([
        ang_t[:, None, None, :].expand(frames, height, width, n_t),
        ang_h[None, :, None, :].expand(frames, height, width, n_h),
        ang_w[None, None, :, :].expand(frames, height, width, n_w),
    ], dim=-1).reshape(frames * height * width, head_dim // 2)
    return torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1).contiguous()


def _partial_sum(part: torch.Tensor, D: int):
    s = part.view(-1, 2, D).sum(0)
    return s[0], s[1]


class ProducerFunction(torch.autograd.Function):
    """apply(proj [B,L,ld], rope [L,F/2,2], ln_w [H,F], ln_b [H,F], H, K,
    base_lr[, eps]) -> (XQ, XK, XV, XU [B,H,NC,K,F] in proj's dtype,
    lr [B,H,NC,K] fp32).  Differentiable wrt proj, ln_w and ln_b."""

    @staticmethod
    def forward(ctx, proj, rope, ln_w, ln_b, H: int, K: int, base_lr: float, eps: float = RECON_EPS):
        if proj.dim() != 3:
            raise ValueError(f"proj must be [B,L,ld], got {tuple(proj.shape)}")
        B, L, ld = proj.shape
        F = ln_w.shape[-1]
        if tuple(ln_w.shape) != (H, F) or tuple(ln_b.shape) != (H, F):
            raise ValueError(f"ttt norm weight/bias must be [H,F]={(H, F)}")
        if tuple(rope.shape) != (L, F // 2, 2):
            raise ValueError(f"rope table must be [L,F/2,2]={(L, F // 2, 2)}, got {tuple(rope.shape)}")
        dev = check_device(proj, rope, ln_w, ln_b)
        code = dtype_code(proj.dtype)
        pj = proj.contiguous()
        rp = rope.to(torch.float32).contiguous()
        lw, lb = ln_w.detach().to(torch.float32).contiguous(), ln_b.detach().to(torch.float32).contiguous()
        NC = L // K
        outs = [torch.empty((B, H, NC, K, F), device=dev, dtype=proj.dtype) for _ in range(4)]
        lr = torch.empty((B, H, NC, K), device=dev, dtype=torch.float32)
        lib = _lib.load()
        with torch.cuda.device(dev):
            st = lib.ttt_qkvu_producer_fwd(ptr(pj), ld, ptr(rp), ptr(lw), ptr(lb), B, L, H, K, F, float(base_lr),
                                           float(eps), code, *(ptr(t) for t in outs), ptr(lr), stream_of(dev))
        _lib.check(st, "ttt_qkvu_producer_fwd")
        ctx.save_for_backward(pj, rp, lw, lb)
        ctx.shape, ctx.base_lr, ctx.eps = (B, L, H, K, F, ld), float(base_lr), float(eps)
        ctx.dtypes = (ln_w.dtype, ln_b.dtype)
        return (*outs, lr)

    @staticmethod
    def backward(ctx, dXQ, dXK, dXV, dXU, dlr):
        pj, rp, lw, lb = ctx.saved_tensors
        B, L, H, K, F, ld = ctx.shape
        dev = pj.device
        code = dtype_code(pj.dtype)

        def act(g):
            if g is None:
                return torch.zeros((B, H, L // K, K, F), device=dev, dtype=pj.dtype)
            return g.to(pj.dtype).contiguous()

        gq, gk, gv, gu = (act(g) for g in (dXQ, dXK, dXV, dXU))
        gl = dlr.to(torch.float32).contiguous() if dlr is not None else None
        dproj = torch.empty_like(pj)
        lib = _lib.load()
        part = torch.empty(lib.ttt_layer_io_partial_bytes(B, L, H, F) // 4, device=dev, dtype=torch.float32)
        with torch.cuda.device(dev):
            st = lib.ttt_qkvu_producer_bwd(ptr(pj), ld, ptr(rp), ptr(lw), ptr(lb), ptr(gq), ptr(gk), ptr(gv), ptr(gu),
                                           ptr(gl) if gl is not None else None, B, L, H, K, F, ctx.base_lr, ctx.eps,
                                           code, ptr(dproj), ptr(part), part.numel() * 4, stream_of(dev))
        _lib.check(st, "ttt_qkvu_producer_bwd")
        dw, db = _partial_sum(part, H * F)
        return (dproj, None, dw.view(H, F).to(ctx.dtypes[0]), db.view(H, F).to(ctx.dtypes[1]), None, None, None,
                None)


class PostNormFunction(torch.autograd.Function):
    """apply(XQW [B,H,NC,K,F], gamma [D], beta [D][, eps]) -> [B, L, D] in
    XQW's dtype: the caller's permute(0,2,3,1,4) + reshape, then LayerNorm
    over D.  Differentiable wrt XQW, gamma and beta."""

    @staticmethod
    def forward(ctx, XQW, gamma, beta, eps: float = POST_NORM_EPS):
        if XQW.dim() != 5:
            raise ValueError(f"XQW must be [B,H,NC,K,F], got {tuple(XQW.shape)}")
        B, H, NC, K, F = XQW.shape
        D, L = H * F, NC * K
        if gamma.numel() != D or beta.numel() != D:
            raise ValueError(f"post-norm weight/bias must have {D} elements")
        dev = check_device(XQW, gamma, beta)
        code = dtype_code(XQW.dtype)
        x = XQW.contiguous()
        g, b = gamma.detach().to(torch.float32).contiguous(), beta.detach().to(torch.float32).contiguous()
        out = torch.empty((B, L, D), device=dev, dtype=XQW.dtype)
        stats = torch.empty((B * L, 2), device=dev, dtype=torch.float32)
        lib = _lib.load()
        with torch.cuda.device(dev):
            st = lib.ttt_post_norm_fwd(ptr(x), ptr(g), ptr(b), B, L, H, K, F, float(eps), code, ptr(out), ptr(stats),
                                       stream_of(dev))
        _lib.check(st, "ttt_post_norm_fwd")
        ctx.save_for_backward(x, g, stats)
        ctx.shape = (B, H, NC, K, F)
        ctx.dtypes = (gamma.dtype, beta.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        x, g, stats = ctx.saved_tensors
        B, H, NC, K, F = ctx.shape
        D, L = H * F, NC * K
        dev = x.device
        code = dtype_code(x.dtype)
        do = dout.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        lib = _lib.load()
        part = torch.empty(lib.ttt_layer_io_partial_bytes(B, L, H, F) // 4, device=dev, dtype=torch.float32)
        with torch.cuda.device(dev):
            st = lib.ttt_post_norm_bwd(ptr(x), ptr(g), ptr(stats), ptr(do), B, L, H, K, F, code, ptr(dx), ptr(part),
                                       part.numel() * 4, stream_of(dev))
        _lib.check(st, "ttt_post_norm_bwd")
        dg, db = _partial_sum(part, D)
        return dx, dg.to(ctx.dtypes[0]), db.to(ctx.dtypes[1]), None


__all__ = ["ProducerFunction", "PostNormFunction", "rope_table", "RECON_EPS", "POST_NORM_EPS"]
