"""The TTT layer stack and forecaster on the HIP path: the caller side of the
inner loop, as TTTForecaster / TTTWrapper / TTTMLP / TTTLinear use it
(forecast.py:79-99, ttt_layer.py:20-565), built on this package's kernels.

Per layer call, for hidden states x [B, L, D] (D = H*F):
  1. one projection GEMM x @ [Wq; Wk; Wv; Wu; w_lr]^T + [bq; bk; bv; bu; b_lr]
     (hipBLASLt through torch), the H lr-gate logits padded to an aligned row
     width (ttt_layer.py:141-148, 151-163); its weight gradient is split over
     row blocks (_ProjectionFunction);
  2. ProducerFunction: L2 norm, RoPE, reconstruction target and lr, written
     in the inner loop's [B,H,NC,K,F] / [B,H,NC,K] layouts (ttt_layer.py:261-309);
  3. the inner loop with eta expanded on chip from lr by the layer's rule
     eta[i][j] = lr[j]/K (ttt_layer.py:309): TTTMLPFunction (+ the memory-cache
     combiner, ttt_layer.py:453-565) or TTTLinearFunction (:383-421);
  4. PostNormFunction (permute + reshape + post_norm, ttt_layer.py:349,
     563-564) and the `wo` GEMM (:350).  A caller that reads only the last
     token (the forecaster's head, forecast.py:97-98) asks for it alone:
     step 4 then runs on the last mini-batch and `wo` on its last row, which
     gives that token's output and every gradient unchanged (the other rows'
     outputs are never read, so their gradients are exact zeros).

Parameter names and shapes are the reference's (wq ... wu, wo,
learnable_ttt_lr_weight [H,1,D], learnable_ttt_lr_bias [H,1],
ttt_norm_weight/bias [H,F], post_norm, W1/b1/W2/b2), so a reference state
dict loads unchanged.  Shapes the layer takes (ModelConfig raises ValueError
for others): head dim F = model_dim / num_heads in {32, 64} (the producer,
post-norm and memory-cache kernels), model_dim <= 1024, and a mini-batch
size K that is a multiple of 16 up to 64.  The inner loop itself runs any
shape on the general-shape kernels; K = 16 with F in {32, 64} (and the MLP's
hidden width F, as TTTMLP builds it) runs on the specialised ones."""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as Fn
from torch import nn

from .layer_io import POST_NORM_EPS, RECON_EPS, PostNormFunction, ProducerFunction, rope_table
from .linear import TTTLinearFunction
from .memo import mlp_memo_combine
from .mlp import LN_EPS, TTTMLPFunction

MAX_MODEL_DIM = 1024  # H * F, the widest row the producer / post-norm kernels take


def _row_blocks(rows: int, target: int) -> int:
    """The largest power of two S <= 16 dividing `rows` with rows / S >= target."""
    s = 1
    while s < 16 and rows % (2 * s) == 0 and rows // (2 * s) >= target:
        s *= 2
    return s


class _ProjectionFunction(torch.autograd.Function):
    """apply(x [R, Din], w [N, Din], b [N]) -> x w^T + b, all in one dtype.

    The backward's weight gradient dy^T x contracts over all R = B*L rows into
    an N x Din output of a few hundred 64x64 tiles, too few to fill the GPU
    with one long contraction each; it is formed instead as S row-block
    products (one batched GEMM) summed in fp32 (in the input's own type when
    that is wider).  The bias gradient is the column sum of dy, taken over row
    blocks the same way."""

    @staticmethod
    def forward(ctx, x, w, b):
        ctx.save_for_backward(x, w)
        return torch.addmm(b, x, w.t())

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        R, N = dy.shape
        dy = dy.contiguous()
        dx = dy @ w if ctx.needs_input_grad[0] else None
        acc = torch.float32 if dy.element_size() < 4 else dy.dtype  # 16-bit inputs summed in fp32
        s = _row_blocks(R, 1024)
        dw = torch.bmm(dy.view(s, R // s, N).transpose(1, 2), x.view(s, R // s, -1)).sum(0, dtype=acc)
        s = 64 if R % 64 == 0 else 1
        db = dy.view(s, R // s, N).sum(1, dtype=acc).sum(0)
        return dx, dw.to(w.dtype), db.to(w.dtype)


def projection(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """Fn.linear(x, weight, bias) over the last dim of x through
    _ProjectionFunction, in the autocast dtype when autocast is on."""
    dt = torch.get_autocast_dtype(x.device.type) if torch.is_autocast_enabled(x.device.type) else x.dtype
    y = _ProjectionFunction.apply(x.reshape(-1, x.shape[-1]).to(dt), weight.to(dt), bias.to(dt))
    return y.view(*x.shape[:-1], weight.shape[0])


def _padded_width(n: int) -> int:
    """Row width of the fused projection: a multiple of 128 where that adds
    at most an eighth (the GEMM then tiles without a ragged edge), else of 8."""
    n128 = -(-n // 128) * 128
    return n128 if 8 * (n128 - n) <= n else -(-n // 8) * 8


@dataclass
class ModelConfig:
    """forecast.py:31-64 (the fields the layer and forecaster read)."""
    seq_len: int = 384
    model_dim: int = 128
    num_heads: int = 4
    num_layers: int = 1
    ssm_layer: str = "ttt_linear"
    layer_norm_eps: float = 1e-6
    mini_batch_size: int = 64
    ttt_base_lr: float = 0.1
    mem_cache_segment_n_mini_batches: int = 2
    mem_cache_max_segments: int = 4
    rope_theta: float = 10000.0
    scan_checkpoint_group_size: int = 16
    latent_height: int = 1
    latent_width: int = 1
    theta: float = 10000.0
    compressed_num_frames: Optional[int] = None

    def __post_init__(self):
        if self.compressed_num_frames is None:
            self.compressed_num_frames = self.seq_len
        if self.model_dim % self.num_heads:
            raise ValueError("model_dim must be a multiple of num_heads")
        if self.seq_len % self.mini_batch_size:
            raise ValueError("seq_len must be a multiple of mini_batch_size")
        if (self.model_dim // self.num_heads) % 2:
            raise ValueError("RoPE needs an even head dim")
        # the fused producer / post-norm kernels and the memory-cache combiner
        # take head dims 32 and 64 and model widths up to 1024; the inner loop
        # takes mini-batches of 16 to 64 tokens in steps of 16
        F = self.model_dim // self.num_heads
        if F not in (32, 64):
            raise ValueError(f"head dim model_dim/num_heads = {F}: this build's layer kernels take 32 or 64")
        if self.model_dim > MAX_MODEL_DIM:
            raise ValueError(f"model_dim {self.model_dim} > {MAX_MODEL_DIM}, the widest the layer kernels take")
        if self.mini_batch_size % 16 or not 16 <= self.mini_batch_size <= 64:
            raise ValueError(f"mini_batch_size {self.mini_batch_size}: a multiple of 16 from 16 to 64 is needed")


class TTTLayerBase(nn.Module):
    """Projections, lr gate, TTT LayerNorm, post-norm and output projection
    (TTTBase, ttt_layer.py:60-139), with the fused producer/consumer."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        self.width = config.model_dim
        self.num_heads = config.num_heads
        self.head_dim = config.model_dim // config.num_heads
        self.mini_batch_size = config.mini_batch_size
        self.ttt_base_lr = config.ttt_base_lr
        self.scan_checkpoint_group_size = config.scan_checkpoint_group_size
        D, H, F = self.width, self.num_heads, self.head_dim
        self.wq = nn.Linear(D, H * F, bias=True)
        self.wk = nn.Linear(D, H * F, bias=True)
        self.wv = nn.Linear(D, H * F, bias=True)
        self.wo = nn.Linear(D, H * F, bias=True)
        self.wu = nn.Linear(D, H * F, bias=True)
        self.learnable_ttt_lr_weight = nn.Parameter(torch.normal(0, 0.02, size=(H, 1, D)))
        self.learnable_ttt_lr_bias = nn.Parameter(torch.zeros(H, 1))
        self.ttt_norm_weight = nn.Parameter(torch.ones(H, F))
        self.ttt_norm_bias = nn.Parameter(torch.zeros(H, F))
        self.post_norm = nn.LayerNorm(D, eps=1e-6)
        # zero rows that pad the fused projection to its row width (not
        # parameters, not in the state dict)
        pad = _padded_width(4 * D + H) - (4 * D + H)
        self.register_buffer("_proj_pad_w", torch.zeros(pad, D), persistent=False)
        self.register_buffer("_proj_pad_b", torch.zeros(pad), persistent=False)

    def init_weights(self):
        """ttt_layer.py:81-89"""
        for lin in (self.wq, self.wk, self.wv, self.wo, self.wu):
            nn.init.normal_(lin.weight, mean=0.0, std=0.02)
        self.post_norm.reset_parameters()
        nn.init.ones_(self.ttt_norm_weight)
        nn.init.zeros_(self.ttt_norm_bias)
        nn.init.normal_(self.learnable_ttt_lr_weight, mean=0.0, std=0.02)
        nn.init.zeros_(self.learnable_ttt_lr_bias)

    def _fused_projection(self, x: torch.Tensor) -> torch.Tensor:
        """[B, L, ld]: XQ | XK | XV | XU | lr logits | zero padding (ld a
        multiple of 8, of 128 where that costs little), one GEMM instead of
        five (ttt_layer.py:141-163)."""
        H, D = self.num_heads, self.width
        w = [self.wq.weight, self.wk.weight, self.wv.weight, self.wu.weight, self.learnable_ttt_lr_weight.view(H, D)]
        b = [self.wq.bias, self.wk.bias, self.wv.bias, self.wu.bias, self.learnable_ttt_lr_bias.view(H)]
        if self._proj_pad_w.shape[0]:
            w.append(self._proj_pad_w.to(self.wq.weight.dtype))
            b.append(self._proj_pad_b.to(self.wq.bias.dtype))
        return projection(x, torch.cat(w, 0), torch.cat(b, 0))

    def process_input(self, x: torch.Tensor, rope: torch.Tensor):
        """(XQ, XK, XV, XU, lr) in the inner loop's layouts (ttt_layer.py:261-329)."""
        B, L, _ = x.shape
        proj = self._fused_projection(x)
        return ProducerFunction.apply(proj, rope[:L], self.ttt_norm_weight, self.ttt_norm_bias, self.num_heads,
                                      self.mini_batch_size, float(self.ttt_base_lr), RECON_EPS)

    def ttt(self, XQ, XK, XV, XU, lr):
        raise NotImplementedError

    def forward(self, x: torch.Tensor, rope: torch.Tensor, last_only: bool = False):
        """[B, L, D], or with last_only the last token's output [B, D]."""
        if x.size(1) % self.mini_batch_size:
            raise ValueError("sequence length must be a multiple of the mini-batch size")
        XQ, XK, XV, XU, lr = self.process_input(x, rope)
        out = self.ttt(XQ, XK, XV, XU, lr)                               # [B,H,NC,K,F]
        if last_only:
            h = PostNormFunction.apply(out[:, :, -1:].contiguous(), self.post_norm.weight, self.post_norm.bias,
                                       POST_NORM_EPS)                    # [B, K, D]
            return self.wo(h[:, -1])
        h = PostNormFunction.apply(out, self.post_norm.weight, self.post_norm.bias, POST_NORM_EPS)
        return self.wo(h)


class TTTLinear(TTTLayerBase):
    """ttt_layer.py:360-421"""

    def __init__(self, config: ModelConfig):
        super().__init__(config)
        H, F = self.num_heads, self.head_dim
        self.W1 = nn.Parameter(torch.normal(0, 0.02, size=(H, F, F)))
        self.b1 = nn.Parameter(torch.zeros(H, 1, F))

    def init_weights(self):
        super().init_weights()
        nn.init.normal_(self.W1, mean=0.0, std=0.02)
        nn.init.zeros_(self.b1)

    def ttt(self, XQ, XK, XV, XU, lr):
        B, NC = XQ.shape[0], XQ.shape[2]
        G = min(max(self.scan_checkpoint_group_size, 1), NC)
        W1 = self.W1.unsqueeze(0).expand(B, -1, -1, -1)
        b1 = self.b1.unsqueeze(0).expand(B, -1, -1, -1)
        return TTTLinearFunction.apply(self.ttt_norm_weight, self.ttt_norm_bias, W1, b1, XQ, XV, XK, lr, G, LN_EPS,
                                       "layer")


class TTTMLP(TTTLayerBase):
    """ttt_layer.py:424-565: the two-layer fast-weight MLP (hidden width F)
    and its memory-cache combiner over segments of M mini-batches."""

    def __init__(self, config: ModelConfig):
        super().__init__(config)
        H, F = self.num_heads, self.head_dim
        self.W1 = nn.Parameter(torch.normal(0, 0.02, size=(H, F, F)))
        self.b1 = nn.Parameter(torch.zeros(H, 1, F))
        self.W2 = nn.Parameter(torch.normal(0, 0.02, size=(H, F, F)))
        self.b2 = nn.Parameter(torch.zeros(H, 1, F))

    def init_weights(self):
        super().init_weights()
        nn.init.normal_(self.W1, mean=0.0, std=0.02)
        nn.init.zeros_(self.b1)
        nn.init.normal_(self.W2, mean=0.0, std=0.02)
        nn.init.zeros_(self.b2)

    def ttt(self, XQ, XK, XV, XU, lr):
        B, NC = XQ.shape[0], XQ.shape[2]
        G = min(max(self.scan_checkpoint_group_size, 1), NC)
        M = self.config.mem_cache_segment_n_mini_batches
        st = [p.unsqueeze(0).expand(B, -1, -1, -1) for p in (self.W1, self.b1, self.W2, self.b2)]
        out, W1m, b1m, W2m, b2m = TTTMLPFunction.apply(self.ttt_norm_weight, self.ttt_norm_bias, *st, XQ, XV, XK, lr,
                                                       G, M, LN_EPS, "layer")
        if M and math.ceil(NC / M) > 1:
            out = mlp_memo_combine(XQ, XK, XU, out, W1m, b1m, W2m, b2m, self.ttt_norm_weight, self.ttt_norm_bias, M)
        return out


class TTTWrapper(nn.Module):
    """ttt_layer.py:20-57: the layer and its rotary table."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        if config.ssm_layer == "ttt_linear":
            self.ttt = TTTLinear(config)
        elif config.ssm_layer == "ttt_mlp":
            self.ttt = TTTMLP(config)
        else:
            raise TypeError(f"no ttt layer of type {config.ssm_layer}")
        self.register_buffer("rope", self._rope(), persistent=False)

    def _rope(self):
        c = self.config
        return rope_table(c.model_dim // c.num_heads, c.compressed_num_frames, c.latent_height, c.latent_width,
                          c.rope_theta)

    def init_freqs(self):
        self.rope.copy_(self._rope())

    def forward(self, x: torch.Tensor, seq_metadata=None, last_only: bool = False):
        return self.ttt(x, self.rope, last_only)


class TTTForecaster(nn.Module):
    """forecast.py:79-99: in_proj -> TTT layer -> head on the last token."""

    def __init__(self, config: ModelConfig, d_in: int, d_out: int, pred_len: int):
        super().__init__()
        self.pred_len, self.d_out = pred_len, d_out
        self.in_proj = nn.Linear(d_in, config.model_dim)
        self.ttt = TTTWrapper(config)
        self.ttt.init_freqs()
        self.head = nn.Linear(config.model_dim, pred_len * d_out)

    def forward(self, seq_x: torch.Tensor) -> torch.Tensor:
        h = projection(seq_x, self.in_proj.weight, self.in_proj.bias)  # self.in_proj(seq_x)
        h = self.ttt(h, last_only=True)  # the head reads h[:, -1] only
        out = self.head(h)
        return out.view(seq_x.size(0), self.pred_len, self.d_out)


__all__ = ["ModelConfig", "TTTLinear", "TTTMLP", "TTTWrapper", "TTTForecaster"]
