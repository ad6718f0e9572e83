"""Pins for the layer/forecaster oracle (oracle/ttt_layer_oracle.py): each
restated function against a library routine, a closed form or an invariant
that a plausible slip (a dropped term, the biased instead of the unbiased
std, a wrong pair order or sign in the rotation, a swapped share of the head
dim) breaks.  CPU only."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ttt_layer_oracle as LO
from oracle import ttt_oracle as O


def _rand(*shape, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


def test_l2_normalize_is_the_library_routine():
    x = _rand(3, 5, 4, 16)
    x[0, 0, 0] = 0.0  # a zero row: the eps clamp, no NaN
    assert torch.allclose(LO.l2_normalize(x), F.normalize(x, p=2, dim=-1), rtol=0, atol=1e-15)
    assert torch.equal(LO.l2_normalize(x)[0, 0, 0], torch.zeros(16, dtype=x.dtype))


@pytest.mark.parametrize("F_", [32, 64])
def test_rope_freqs_closed_form(F_):
    T = 300
    fr = LO.rope_freqs(F_, 1, 1, T)
    assert fr.shape == (T, F_ // 2) and fr.dtype == torch.complex64
    assert torch.allclose(fr.abs(), torch.ones_like(fr.abs()), atol=1e-6)
    nt = F_ // 8  # pairs of the frame share (F/4 features)
    # height = width = 1: the row and column shares see position 0 -> no rotation
    assert torch.equal(fr[:, nt:], torch.ones_like(fr[:, nt:]))
    t = torch.arange(T, dtype=torch.float64)[:, None]
    p = torch.arange(nt, dtype=torch.float64)[None, :]
    ang = t * 10000.0 ** (-2 * p / (F_ // 4))
    assert torch.allclose(fr[:, :nt].real.double(), torch.cos(ang), atol=2e-4)
    assert torch.allclose(fr[:, :nt].imag.double(), torch.sin(ang), atol=2e-4)


def test_rope_freqs_3d_layout():
    """(t h w) flattening with t outermost; the row share rotates with h."""
    F_, T, Hl, Wl = 32, 3, 2, 4
    fr = LO.rope_freqs(F_, Hl, Wl, T)
    nt, nh = F_ // 8, (F_ // 8 * 3) // 2
    fr = fr.view(T, Hl, Wl, F_ // 2)
    assert torch.equal(fr[:, 0, 0, nt:], torch.ones_like(fr[:, 0, 0, nt:]))
    assert torch.equal(fr[1, 1, 0, :nt], fr[1, 0, 3, :nt])          # the frame share ignores h, w
    assert not torch.equal(fr[0, 1, 0, nt:nt + nh], fr[0, 0, 0, nt:nt + nh])
    assert torch.equal(fr[0, 0, 2, nt:nt + nh], fr[0, 0, 0, nt:nt + nh])  # the row share ignores w


def test_product_rope_table_matches_the_oracle():
    """The product's table (cos, sin in fp32) is the oracle's complex table."""
    from ttt_amd.layer_io import rope_table
    for F_, T, Hl, Wl in ((64, 512, 1, 1), (32, 64, 1, 1), (32, 3, 2, 4)):
        tab = rope_table(F_, T, Hl, Wl)
        fr = LO.rope_freqs(F_, Hl, Wl, T)
        assert torch.allclose(tab[..., 0], fr.real, rtol=0, atol=1e-6)
        assert torch.allclose(tab[..., 1], fr.imag, rtol=0, atol=1e-6)


def test_apply_rope_is_a_pairwise_rotation():
    B, L, H, F_ = 2, 40, 3, 32
    x = _rand(B, L, H, F_, seed=1)
    fr = LO.rope_freqs(F_, 1, 1, L)
    y = LO.apply_rope(x, fr)
    c, s = fr.real.double()[None, :, None, :], fr.imag.double()[None, :, None, :]
    x0, x1 = x[..., 0::2], x[..., 1::2]
    assert torch.allclose(y[..., 0::2], x0 * c - x1 * s, atol=1e-12)
    assert torch.allclose(y[..., 1::2], x0 * s + x1 * c, atol=1e-12)
    assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), atol=1e-12)


def test_apply_rope_relative_positions():
    """<R_m q, R_n k> depends on m - n only."""
    F_, L = 64, 64
    fr = LO.rope_freqs(F_, 1, 1, L)
    q, k = _rand(F_, seed=2), _rand(F_, seed=3)
    xs = torch.zeros(1, L, 2, F_, dtype=torch.float64)
    xs[0, :, 0], xs[0, :, 1] = q, k
    y = LO.apply_rope(xs, fr)
    dots = [(y[0, m, 0] @ y[0, n, 1]).item() for m, n in ((5, 2), (20, 17), (60, 57))]
    assert max(dots) - min(dots) < 1e-5 * max(1.0, abs(dots[0]))
    assert abs((y[0, 5, 0] @ y[0, 2, 1]).item() - (y[0, 5, 0] @ y[0, 3, 1]).item()) > 1e-3


def test_recon_target_unbiased_std():
    B, L, H, F_ = 2, 7, 3, 16
    XV, XK = _rand(B, L, H, F_, seed=4), _rand(B, L, H, F_, seed=5)
    ones, zeros = torch.ones(H, F_, dtype=torch.float64), torch.zeros(H, F_, dtype=torch.float64)
    r = LO.recon_target(XV, XK, ones, zeros) - XK
    d = XV - XK
    sd = d.std(dim=-1, keepdim=True)  # unbiased: the library's default
    assert torch.allclose(r.mean(-1), torch.zeros_like(r.mean(-1)), atol=1e-12)
    assert torch.allclose(r.std(dim=-1, keepdim=True), sd / (sd + LO.RECON_EPS), atol=1e-12)
    w, b = _rand(H, F_, seed=6), _rand(H, F_, seed=7)
    ref = w * (d - d.mean(-1, keepdim=True)) / (d.std(-1, keepdim=True) + 1e-8) + b + XK
    assert torch.allclose(LO.recon_target(XV, XK, w, b), ref, atol=1e-12)


def test_lr_gate_scalar_loops():
    B, NC, K, D, H, Fh, base = 2, 3, 4, 6, 2, 3, 0.05
    X = _rand(B, NC, K, D, seed=8)
    w, b = _rand(H, 1, D, seed=9), _rand(H, 1, seed=10)
    lr = LO.lr_gate(X, w, b, base, Fh)
    for bb in range(B):
        for h in range(H):
            for n in range(NC):
                for k in range(K):
                    z = sum(X[bb, n, k, c].item() * w[h, 0, c].item() for c in range(D)) + b[h, 0].item()
                    assert abs(lr[bb, h, n, k].item() - base / (1 + math.exp(-z)) / Fh) < 1e-14


def _layer_params(D, H, Fh, FF, kind, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=0.2: sc * torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    p = {}
    for n in ("wq", "wk", "wv", "wu", "wo"):
        p[n + ".weight"], p[n + ".bias"] = r(D, D), r(D, sc=0.05)
    p["learnable_ttt_lr_weight"], p["learnable_ttt_lr_bias"] = r(H, 1, D), r(H, 1, sc=0.5)
    p["ttt_norm_weight"], p["ttt_norm_bias"] = 1 + r(H, Fh, sc=0.1), r(H, Fh, sc=0.1)
    p["post_norm.weight"], p["post_norm.bias"] = 1 + r(D, sc=0.1), r(D, sc=0.1)
    p["W1"], p["b1"] = r(H, Fh, FF, sc=0.1), r(H, 1, FF, sc=0.05)
    if kind == "ttt_mlp":
        p["W2"], p["b2"] = r(H, FF, Fh, sc=0.1), r(H, 1, Fh, sc=0.05)
    return p


def test_process_input_eta_is_the_layer_rule():
    B, L, H, Fh, K = 1, 32, 2, 16, 16
    D = H * Fh
    p = _layer_params(D, H, Fh, Fh, "ttt_mlp", 11)
    x = _rand(B, L, D, seed=12)
    XQ, XK, XV, XU, eta, lr = LO.process_input(p, x, LO.rope_freqs(Fh, 1, 1, L), H, K, 0.1)
    assert XQ.shape == (B, H, L // K, K, Fh) and lr.shape == (B, H, L // K, K)
    assert torch.allclose(eta, (lr / K)[..., None, :].expand_as(eta), atol=0)
    lr2 = LO.lr_gate(x.view(B, L // K, K, D), p["learnable_ttt_lr_weight"], p["learnable_ttt_lr_bias"], 0.1, Fh)
    assert torch.allclose(lr, lr2, atol=1e-15)
    # unit norm after L2 + rotation
    assert torch.allclose(XQ.norm(dim=-1), torch.ones_like(XQ.norm(dim=-1)), atol=1e-12)


@pytest.mark.parametrize("kind,M", [("ttt_mlp", 0), ("ttt_linear", 0)])
def test_layer_directional_derivatives(kind, M):
    """Autograd of the whole layer (projections, producer, inner loop,
    post-norm, wo) against central finite differences along random
    directions in every parameter and the input at once.  Without the memory
    cache (M = 0): with it the reference's gradient is by design not the
    derivative (memo states, cached readouts and cached summaries are
    detached, ttt_layer.py:521,543,559), and the combiner's own gradient
    rules are pinned in test_oracle.py."""
    B, L, H, Fh, K = 1, 32, 2, 16, 16
    D = H * Fh
    p = _layer_params(D, H, Fh, Fh, kind, 13)
    x = _rand(B, L, D, seed=14)
    fr = LO.rope_freqs(Fh, 1, 1, L)
    dout = _rand(B, L, D, seed=15)
    names = sorted(p)

    def f(x_, *vals):
        q = dict(zip(names, vals))
        return (LO.layer_forward(q, x_, fr, H, K, 0.3, kind, 1, M) * dout).sum()

    vals = [p[n].clone().requires_grad_(True) for n in names]
    xg = x.clone().requires_grad_(True)
    f(xg, *vals).backward()
    for seed in (16, 17):
        g = torch.Generator().manual_seed(seed)
        dirs = [torch.randn(v.shape, generator=g, dtype=torch.float64) for v in vals]
        dx = torch.randn(x.shape, generator=g, dtype=torch.float64)
        ana = (xg.grad * dx).sum().item() + sum((v.grad * d).sum().item() for v, d in zip(vals, dirs)
                                                if v.grad is not None)
        h = 1e-5
        with torch.no_grad():
            fp = f(x + h * dx, *(v + h * d for v, d in zip(vals, dirs))).item()
            fm = f(x - h * dx, *(v - h * d for v, d in zip(vals, dirs))).item()
        num = (fp - fm) / (2 * h)
        assert abs(ana - num) <= 1e-6 * max(1.0, abs(num)), (ana, num)


def test_row_split_projection_matches_linear():
    """The model's projection (weight gradient as a sum of row-block
    products, bias gradient by row blocks) against torch's linear on the CPU:
    the same output and gradients in fp64, at row counts with 16, 4 and 1 row
    blocks, with and without an input gradient."""
    from ttt_amd.model import _padded_width, _ProjectionFunction, _row_blocks, projection
    assert (_row_blocks(16384, 1024), _row_blocks(4096, 1024), _row_blocks(1000, 1024)) == (16, 4, 1)
    assert _padded_width(1028) == 1152 and _padded_width(516) == 520 and _padded_width(3084) == 3200
    for rows, din, dout, xgrad in ((16384, 7, 64, False), (4096, 32, 130, True), (1000, 16, 24, True)):
        x = _rand(rows, din, seed=rows).requires_grad_(xgrad)
        w = _rand(dout, din, seed=1).requires_grad_(True)
        b = _rand(dout, seed=2).requires_grad_(True)
        dy = _rand(rows, dout, seed=3)
        y = _ProjectionFunction.apply(x, w, b)
        y.backward(dy)
        mine = (y.detach(), w.grad.clone(), b.grad.clone(), x.grad.clone() if xgrad else None)
        w.grad = b.grad = x.grad = None
        y_ref = F.linear(x, w, b)
        y_ref.backward(dy)
        assert torch.allclose(mine[0], y_ref.detach(), rtol=1e-12, atol=1e-12)
        assert torch.allclose(mine[1], w.grad, rtol=1e-10, atol=1e-9)
        assert torch.allclose(mine[2], b.grad, rtol=1e-10, atol=1e-9)
        if xgrad:
            assert torch.allclose(mine[3], x.grad, rtol=1e-12, atol=1e-12)
    # projection() keeps the leading dims
    x3 = _rand(2, 8, 5, seed=9)
    assert projection(x3, _rand(3, 5, seed=10), _rand(3, seed=11)).shape == (2, 8, 3)


def _producer_case(seed=5, B=2, L=32, H=3, Fh=32, K=16):
    XQ, XK, XV, XU = (_rand(B, L, H, Fh, seed=seed + i) for i in range(4))
    logits = _rand(B, L, H, seed=seed + 4)
    freqs = LO.rope_freqs(Fh, 1, 1, L)
    ones, zeros = torch.ones(H, Fh, dtype=torch.float64), torch.zeros(H, Fh, dtype=torch.float64)
    out = LO.producer(XQ, XK, XV, XU, logits, freqs, ones, zeros, K, 1.0)
    return (XQ, XK, XV, XU), out, K


def test_producer_target_is_built_on_the_rotated_xk():
    """ttt_layer.py:279-302 rotates XK first and builds the reconstruction
    target from the rotated XK.  With ln_w = 1, ln_b = 0 the target minus the
    XK the loop receives is (d - mean d) / (std d + eps), d = XV - XK_out: per
    token and head zero mean and unbiased std sigma / (sigma + 1e-8) = 1 to
    1e-7.  A target built on the unrotated (or unnormalised) XK adds
    XK_l2 - rot(XK_l2) to it, which breaks both at every rotated position."""
    _, (q, k, v, u, lr), K = _producer_case()
    d = v - k                                        # [B, H, NC, K, F]
    mean = d.mean(-1)
    std = d.std(-1, unbiased=True)
    assert float(mean.abs().max()) < 1e-12
    assert float((std - 1).abs().max()) < 1e-7
    # the slip this pins: the target on the L2-normalised but unrotated XK
    (XQ, XK, XV, XU), _, _ = _producer_case()
    B, L, H, Fh = XK.shape
    kl2 = LO.l2_normalize(XK)
    bad = LO.recon_target(XV, kl2, torch.ones(H, Fh, dtype=torch.float64), torch.zeros(H, Fh, dtype=torch.float64))
    bad = bad.transpose(1, 2).reshape(B, H, L // K, K, Fh)
    assert float((bad - k).mean(-1)[:, :, :, 1:].abs().max()) > 1e-3


def test_producer_rotates_xu_like_xq():
    """XU is L2-normalised and rotated with the same table as XQ
    (ttt_layer.py:289-295): at one position both are rotated by the same
    angles, so <XU_out, XQ_out> = <l2(XU), l2(XQ)>, while XU_out differs from
    l2(XU) wherever the angles are not zero (every position but the first).
    An unrotated XU fails the first identity, a missing normalisation both."""
    (XQ, XK, XV, XU), (q, k, v, u, lr), K = _producer_case()
    B, L, H, Fh = XQ.shape
    to_mb = lambda t: t.transpose(1, 2).reshape(B, H, L // K, K, Fh)  # noqa: E731
    ql2, ul2 = to_mb(LO.l2_normalize(XQ)), to_mb(LO.l2_normalize(XU))
    # (the rotary table is fp32, as the reference's: unit modulus to ~1e-7)
    assert torch.allclose((u * q).sum(-1), (ul2 * ql2).sum(-1), rtol=0, atol=1e-6)
    assert torch.allclose(u.norm(dim=-1), torch.ones_like(u[..., 0]), rtol=0, atol=1e-6)
    diff = (u - ul2).norm(dim=-1).reshape(B, H, L)
    assert float(diff[:, :, 0].abs().max()) < 1e-15      # position 0: angle 0
    assert float(diff[:, :, 1:].min()) > 1e-4             # every other position rotated
    # the slip this pins: XU left unrotated gives other inner products
    assert float(((ul2 * q).sum(-1) - (ul2 * ql2).sum(-1)).abs().max()) > 1e-3
