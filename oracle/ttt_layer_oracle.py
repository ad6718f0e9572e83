"""CPU oracle for the caller side of the TTT inner loop: the layer's
producer and consumer, the TTT-MLP / TTT-Linear layer and the forecaster.

TEST INFRASTRUCTURE ONLY.  Plain eager PyTorch on the CPU, imported by
`tests/` and `bench.py`'s CPU baseline as the checker; the product
(`ttt-triton_amd/`) never imports it.  It reads a state dict with the
reference's parameter names (the product model keeps them), so both run on
the same weights.

What it restates (reference file:line):
  l2_normalize        ttt_layer.py:279-281     F.normalize(p=2, dim=-1): x / max(|x|, 1e-12)
  rope_freqs          utils.py:24-68           precompute_freqs_cis_3d (complex64 table)
  apply_rope          utils.py:71-123          reshape_for_broadcast + apply_rotary_emb
  recon_target        ttt_layer.py:227-243     ln_reconstruction_target, unbiased std, eps 1e-8
  lr_gate             ttt_layer.py:151-163     get_eta: sigmoid(x . w_h + b_h) * base_lr / F
  producer            ttt_layer.py:279-304     the above from the projections, reshape_to_mini_batch
                                               (:245-259), lr = sigmoid(logit) * base_lr / F
  process_input       ttt_layer.py:261-329     projections, producer, the row-repeated eta (:306-309)
  mlp_layer_ttt       ttt_layer.py:453-565     ops-path ttt_mlp, memo states after step s*M,
                                               the memory-cache combiner
  linear_layer_ttt    ttt_layer.py:383-421
  layer_forward       ttt_layer.py:337-357     ttt -> post_norm (eps 1e-6) -> wo
  forecaster_forward  forecast.py:94-99        in_proj -> layer -> head(h[:, -1])

How each function is pinned (tests/test_oracle_layer.py):
  l2_normalize        == torch.nn.functional.normalize (library routine)
  rope_freqs          only the first F/8 pairs rotate at height = width = 1 (the
                      h and w shares see position 0); |freqs| = 1; the angle of
                      pair p at frame t is t * theta^(-2p/(F/4)) (closed form)
  apply_rope          == the real 2x2 rotation of each pair; preserves norms;
                      <R_m q, R_n k> depends on m - n only (relative position)
  recon_target        with weight 1 / bias 0: recon - XK has zero mean and
                      unbiased std std/(std + eps); == torch.std-based formula
  lr_gate             == scalar loops over (b, h, token)
  process_input       eta rows all equal lr / K (the layer rule); lr == lr_gate
  layer               autograd == central finite differences along random directions in
                      every parameter and the input (fp64, tiny size, no memo cache: with
                      it the reference's gradient is by design not the derivative; the
                      combiner's gradient rules are pinned with ttt_oracle.memo_combine)
  forecaster          the composition of the above (in_proj, layer, head on the last token)
"""

from __future__ import annotations

import math
from typing import Dict

import torch
import torch.nn.functional as F

from oracle import ttt_oracle as O

RECON_EPS = 1e-8       # ttt_layer.py:230
POST_NORM_EPS = 1e-6   # ttt_layer.py:78
L2_EPS = 1e-12         # torch.nn.functional.normalize default


def l2_normalize(x, eps: float = L2_EPS):
    """x / max(||x||_2, eps) over the last dim.  ttt_layer.py:279-281."""
    n = torch.sqrt((x * x).sum(-1, keepdim=True))
    return x / n.clamp_min(eps)


def rope_freqs(dim: int, height: int, width: int, frames: int, theta: float = 10000.0):
    """Complex [frames*height*width, dim/2] table.  utils.py:24-68: the head
    dim split dim/4 (frames), 3dim/8 (rows), 3dim/8 (columns), each share with
    frequencies theta^(-2i/d), angles position * frequency, (t h w) flattened."""
    dt, dh, dw = dim // 4, dim // 8 * 3, dim // 8 * 3
    ft = 1.0 / (theta ** (torch.arange(0, dt, 2)[: dt // 2].float() / dt))
    fh = 1.0 / (theta ** (torch.arange(0, dh, 2)[: dh // 2].float() / dh))
    fw = 1.0 / (theta ** (torch.arange(0, dw, 2)[: dw // 2].float() / dw))
    at = torch.arange(frames, dtype=torch.float32)[:, None] * ft[None]
    ah = torch.arange(height, dtype=torch.float32)[:, None] * fh[None]
    aw = torch.arange(width, dtype=torch.float32)[:, None] * fw[None]
    ang = torch.cat([at[:, None, None, :].expand(frames, height, width, -1),
                     ah[None, :, None, :].expand(frames, height, width, -1),
                     aw[None, None, :, :].expand(frames, height, width, -1)], dim=-1)
    ang = ang.reshape(frames * height * width, -1)
    return torch.polar(torch.ones_like(ang), ang)


def apply_rope(x, freqs):
    """x [B, L, H, F] rotated pairwise by freqs[:L] (complex [*, F/2]).
    utils.py:97-123 (computed in float, returned in x's dtype when that is
    float32 or float64 -- the reference returns x's dtype)."""
    L = x.shape[1]
    work = torch.float64 if x.dtype == torch.float64 else torch.float32
    xc = torch.view_as_complex(x.to(work).reshape(*x.shape[:-1], -1, 2).contiguous())
    f = freqs[:L].to(xc.dtype).view(1, L, 1, -1)
    return torch.view_as_real(xc * f).flatten(3).to(x.dtype)


def recon_target(XV, XK, ln_w, ln_b, eps: float = RECON_EPS):
    """ln_w * (d - mean d) / (std d + eps) + ln_b + XK, d = XV - XK, unbiased
    std over the head dim; XV, XK [B, L, H, F], ln [H, F].  ttt_layer.py:227-243."""
    d = XV - XK
    mean = d.mean(dim=-1, keepdim=True)
    std = torch.sqrt(((d - mean) ** 2).sum(-1, keepdim=True) / (d.shape[-1] - 1))
    return ln_w[None, None] * ((d - mean) / (std + eps)) + ln_b[None, None] + XK


def lr_gate(X, lr_w, lr_b, base_lr: float, head_dim: int):
    """X [B, NC, K, D], lr_w [H, 1, D], lr_b [H, 1] -> lr [B, H, NC, K]
    (ttt_layer.py:151-163 before its final permute to [..., 1, K])."""
    z = torch.einsum("bnkc,hc->bhnk", X, lr_w[:, 0, :]) + lr_b.view(1, -1, 1, 1)
    return base_lr * torch.sigmoid(z) / head_dim


def producer(XQ, XK, XV, XU, logits, freqs, ln_w, ln_b, K: int, base_lr: float):
    """From the projections XQ, XK, XV, XU [B, L, H, F] and the lr-gate
    logits [B, L, H] to the inner loop's inputs (XQ, XK, XV, XU [B,H,NC,K,F],
    lr [B,H,NC,K]): ttt_layer.py:279-304 and the sigmoid/scale of :160-163."""
    B, L, H, Fh = XQ.shape
    XQ, XK, XU = l2_normalize(XQ), l2_normalize(XK), l2_normalize(XU)
    XQ, XK, XU = apply_rope(XQ, freqs), apply_rope(XK, freqs), apply_rope(XU, freqs)
    XV = recon_target(XV, XK, ln_w, ln_b)
    NC = L // K
    to_mb = lambda t: t.transpose(1, 2).reshape(B, H, NC, K, Fh)  # noqa: E731
    lr = base_lr * torch.sigmoid(logits) / Fh
    return to_mb(XQ), to_mb(XK), to_mb(XV), to_mb(XU), lr.transpose(1, 2).reshape(B, H, NC, K)


def process_input(p: Dict[str, torch.Tensor], x, freqs, H: int, K: int, base_lr: float):
    """(XQ, XK, XV, XU [B,H,NC,K,F], eta [B,H,NC,K,K], lr [B,H,NC,K]).
    ttt_layer.py:261-329 (no text prefix, no multiscene)."""
    B, L, D = x.shape
    Fh = D // H
    lin = lambda n: F.linear(x, p[n + ".weight"], p[n + ".bias"])  # noqa: E731
    XQ, XK, XV, XU = (lin(n).view(B, L, H, Fh) for n in ("wq", "wk", "wv", "wu"))
    NC = L // K
    logits = torch.einsum("blc,hc->blh", x, p["learnable_ttt_lr_weight"][:, 0, :]) + p["learnable_ttt_lr_bias"].view(1, 1, H)
    XQ, XK, XV, XU, lr = producer(XQ, XK, XV, XU, logits, freqs, p["ttt_norm_weight"], p["ttt_norm_bias"], K, base_lr)
    eta = O.eta_from_lr(lr, "layer")
    return XQ, XK, XV, XU, eta, lr


def mlp_layer_ttt(p, XQ, XK, XV, XU, eta, G: int, M: int):
    """TTTMLP.ttt (ttt_layer.py:453-565): the ops-path inner loop, then the
    memory-cache combiner over the states after mini-batches s*M (the
    kernel path's memo, non-differentiable).  Returns [B,H,NC,K,F]."""
    B = XQ.shape[0]
    NC = XQ.shape[2]
    st = [p[n].unsqueeze(0).expand(B, *p[n].shape) for n in ("W1", "b1", "W2", "b2")]
    G = min(max(G, 1), NC)
    out = O.ttt_mlp(XK, XQ, XV, eta, p["ttt_norm_weight"], p["ttt_norm_bias"], *st, G)  # [B,NC,K,H,F]
    out = out.permute(0, 3, 1, 2, 4)
    if M and math.ceil(NC / M) > 1:
        with torch.no_grad():
            full = O.mlp_forward_full(p["ttt_norm_weight"], p["ttt_norm_bias"], *(t.detach() for t in st),
                                      XQ.detach(), XV.detach(), XK.detach(), eta.detach(), G, M=M)
        memo = [full[n + "_memo"] for n in ("W1", "b1", "W2", "b2")]
        out = O.memo_combine(XQ, XK, XU, out, *memo, p["ttt_norm_weight"], p["ttt_norm_bias"], M, dtype=out.dtype)
    return out


def linear_layer_ttt(p, XQ, XK, XV, XU, eta, G: int):
    """TTTLinear.ttt (ttt_layer.py:383-421), ops path.  Returns [B,H,NC,K,F]."""
    B, NC = XQ.shape[0], XQ.shape[2]
    W1 = p["W1"].unsqueeze(0).expand(B, *p["W1"].shape)
    b1 = p["b1"].unsqueeze(0).expand(B, *p["b1"].shape)
    G = min(max(G, 1), NC)
    out = O.ttt_linear(XK, XQ, XV, eta, p["ttt_norm_weight"], p["ttt_norm_bias"], W1, b1, G)
    return out.permute(0, 3, 1, 2, 4)


def layer_forward(p, x, freqs, H: int, K: int, base_lr: float, kind: str, G: int, M: int):
    """TTTBase.forward (ttt_layer.py:337-357): [B, L, D] -> [B, L, D]."""
    B, L, D = x.shape
    XQ, XK, XV, XU, eta, _ = process_input(p, x, freqs, H, K, base_lr)
    if kind == "ttt_mlp":
        out = mlp_layer_ttt(p, XQ, XK, XV, XU, eta, G, M)
    else:
        out = linear_layer_ttt(p, XQ, XK, XV, XU, eta, G)
    h = out.permute(0, 2, 3, 1, 4).reshape(B, L, D)
    h = F.layer_norm(h, (D,), p["post_norm.weight"], p["post_norm.bias"], POST_NORM_EPS)
    return F.linear(h, p["wo.weight"], p["wo.bias"])


def forecaster_forward(sd: Dict[str, torch.Tensor], x, cfg, pred_len: int, d_out: int):
    """TTTForecaster.forward (forecast.py:94-99) on a state dict `sd` with the
    reference's names (in_proj.*, ttt.ttt.*, head.*); cfg has num_heads,
    mini_batch_size, ttt_base_lr, ssm_layer, scan_checkpoint_group_size,
    mem_cache_segment_n_mini_batches, rope_theta, latent_height,
    latent_width, compressed_num_frames."""
    layer = {k[len("ttt.ttt."):]: v for k, v in sd.items() if k.startswith("ttt.ttt.")}
    D = sd["in_proj.weight"].shape[0]
    Fh = D // cfg.num_heads
    freqs = rope_freqs(Fh, cfg.latent_height, cfg.latent_width, cfg.compressed_num_frames, cfg.rope_theta)
    h = F.linear(x, sd["in_proj.weight"], sd["in_proj.bias"])
    h = layer_forward(layer, h, freqs, cfg.num_heads, cfg.mini_batch_size, cfg.ttt_base_lr, cfg.ssm_layer,
                      cfg.scan_checkpoint_group_size, cfg.mem_cache_segment_n_mini_batches)
    out = F.linear(h[:, -1], sd["head.weight"], sd["head.bias"])
    return out.view(x.shape[0], pred_len, d_out)
