"""TTT-Linear HIP kernels vs the CPU oracle (forward, side outputs, backward).

Tolerances: fp32 activations max-abs <= 1e-4 against the ops
path, or, where the tensor's own fp32 evaluation is less exact (the eta
gradient), C_FP32 = 8 times the fp32 oracle's error against fp64
(tests/_util.fp32_bound); bf16 activations with fp32 state rel-L2 <= 2e-2.
The oracle runs in fp64 on the same (bf16-rounded) inputs."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import C_FP32, FP32_ATOL, eta_own_dtype, fp32_bound, max_abs, oracle_linear_grads, rel_l2, to_dev

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _fwd(d, G, want_last=True, want_saved=False):
    from ttt_amd.linear import linear_forward
    g = to_dev(d)
    res = linear_forward(g["ln_w"], g["ln_b"], g["W1"], g["b1"], g["XQ"], g["XV"], g["XK"], g["eta"], G,
                         want_ckpt=True, want_last=want_last, want_saved=want_saved)
    return res if want_saved else res[:3]


def _unpack_saved(saved, B, H, NC, F_):
    """Saved slots -> per mini-batch G, XH, XHB [B,H,NC,16,F] and RSTD, CC, RSB [B,H,NC,16].
    G and XH are token-major tiles in lane order (tile o, lane (g, n), register j
    holds row 4g + j, column 16o + n); XHB is feature-major (token n, feature
    16o + 4g + j)."""
    FT = F_ // 16
    slot = 3 * F_ * 64 + 256
    raw = saved.view(torch.float32).reshape(B, H, NC, slot // 4)
    tiles = raw[..., : 3 * F_ * 16].reshape(B, H, NC, 3, FT, 4, 16, 4)  # [.., part, o, g, n, j]
    tm = tiles.permute(0, 1, 2, 3, 5, 7, 4, 6).reshape(B, H, NC, 3, 16, F_)   # [g, j, o, n]
    fm = tiles.permute(0, 1, 2, 3, 6, 4, 5, 7).reshape(B, H, NC, 3, 16, F_)   # [n, o, g, j]
    stats = raw[..., 3 * F_ * 16:3 * F_ * 16 + 48].reshape(B, H, NC, 3, 16)
    return dict(G=tm[:, :, :, 0], XH=tm[:, :, :, 1], XHB=fm[:, :, :, 2], RSTD=stats[:, :, :, 0],
                CC=stats[:, :, :, 1], RSB=stats[:, :, :, 2])


def test_linear_fwd_saved_buffer():
    """The saved values reproduce the state update and the readout, and saving
    leaves every output unchanged."""
    _say("linear fwd saved buffer fp32")
    B, H, NC, F_ = 2, 2, 6, 64
    d = O.make_inputs(B, H, NC, 16, F_, seed=11, dtype=torch.float32, eta_kind="layer")
    gen = torch.Generator().manual_seed(12)
    d["ln_w"] = 1 + 0.2 * torch.randn(H, F_, generator=gen)
    d["ln_b"] = 0.2 * torch.randn(H, F_, generator=gen)
    out0, (Wc0, bc0), (Wl0, bl0) = _fwd(d, G=4)
    out, (Wc, bc), (Wl, bl), saved = _fwd(d, G=4, want_saved=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out0) and torch.equal(Wl, Wl0) and torch.equal(bl, bl0) and torch.equal(Wc, Wc0)
    sv = {k: v.cpu().double() for k, v in _unpack_saved(saved, B, H, NC, F_).items()}
    XK, XV, XQ = d["XK"].double(), d["XV"].double(), d["XQ"].double()
    e = d["eta"].double()[..., -1, :]                                   # [B,H,NC,K]
    # W_last = W_init - sum_s XK_s^T diag(e_s) G_s ; b_last = b_init - sum_s G_s^T e_s
    dW = torch.einsum("bhstf,bhst,bhsto->bhfo", XK, e, sv["G"])
    assert max_abs(Wl, d["W1"].double() - dW) <= 1e-4
    db = torch.einsum("bhst,bhsto->bho", e, sv["G"]).unsqueeze(2)
    assert max_abs(bl, d["b1"].double() - db) <= 1e-4
    # G from the saved normalised Z1 and its statistics (ops/ttt_utils.py:21-48)
    lw, lb = d["ln_w"].double()[None, :, None, None, :], d["ln_b"].double()[None, :, None, None, :]
    xh = sv["XH"]
    gx = (lw * xh + lb - (XV - XK)) * lw
    G = (gx - gx.mean(-1, keepdim=True) - xh * sv["CC"][..., None]) * sv["RSTD"][..., None]
    assert max_abs(G, sv["G"]) <= 1e-4
    assert max_abs(sv["CC"], (gx * xh).mean(-1)) <= 1e-4
    assert max_abs(xh.mean(-1), torch.zeros_like(sv["RSTD"])) <= 1e-4
    # readout: out = XQ + ln_w * XHB + ln_b, XHB normalised per token
    assert max_abs(out, XQ + lw * sv["XHB"] + lb) <= 1e-4
    assert max_abs(sv["XHB"].pow(2).mean(-1), torch.ones_like(sv["RSB"])) <= 1e-3
    assert bool((sv["RSB"] > 0).all()) and bool((sv["RSTD"] > 0).all())


@pytest.mark.parametrize("kind", ["causal", "layer"])
def test_linear_fwd_fp32_config0(kind):
    """The CPU-runnable small case: B2 H4 T256 (NC16 K16) F64, fp32."""
    _say("linear fwd fp32 config0", kind)
    d = O.make_inputs(2, 4, 16, 16, 64, seed=0, dtype=torch.float32, eta_kind=kind)
    out, (Wc, bc), (Wl, bl) = _fwd(d, G=4)
    torch.cuda.synchronize()
    ref = O.linear_forward_full(*(d[k].double() for k in ("ln_w", "ln_b", "W1", "b1", "XQ", "XV", "XK", "eta")), G=4)
    assert max_abs(out, ref["out"]) <= FP32_ATOL
    assert max_abs(Wl, ref["W1_last"]) <= FP32_ATOL
    assert max_abs(bl, ref["b1_last"]) <= FP32_ATOL
    assert max_abs(Wc, ref["W1_ckpt"]) <= FP32_ATOL
    assert max_abs(bc, ref["b1_ckpt"]) <= FP32_ATOL


def test_linear_fwd_fp32_nonzero_ln_and_bias():
    _say("linear fwd fp32 ln/bias")
    d = O.make_inputs(1, 3, 8, 16, 64, seed=5, dtype=torch.float32)
    gen = torch.Generator().manual_seed(9)
    d["ln_w"] = 1 + 0.2 * torch.randn(3, 64, generator=gen)
    d["ln_b"] = 0.2 * torch.randn(3, 64, generator=gen)
    d["b1"] = 0.1 * torch.randn(1, 3, 1, 64, generator=gen)
    out, _, (Wl, bl) = _fwd(d, G=3)
    ref = O.linear_forward_full(*(d[k].double() for k in ("ln_w", "ln_b", "W1", "b1", "XQ", "XV", "XK", "eta")), G=3)
    assert max_abs(out, ref["out"]) <= FP32_ATOL
    assert max_abs(Wl, ref["W1_last"]) <= FP32_ATOL
    assert max_abs(bl, ref["b1_last"]) <= FP32_ATOL


def test_linear_fwd_f32_headdim32():
    _say("linear fwd fp32 F=32")
    d = O.make_inputs(2, 2, 6, 16, 32, seed=3, dtype=torch.float32)
    out, _, (Wl, _) = _fwd(d, G=2)
    ref = O.linear_forward_full(*(d[k].double() for k in ("ln_w", "ln_b", "W1", "b1", "XQ", "XV", "XK", "eta")), G=2)
    assert max_abs(out, ref["out"]) <= FP32_ATOL
    assert max_abs(Wl, ref["W1_last"]) <= FP32_ATOL


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("kind", ["causal", "layer"])
def test_linear_fwd_16bit(kind, dt):
    _say("linear fwd", dt, kind)
    d = O.make_inputs(2, 3, 32, 16, 64, seed=1, dtype=dt, eta_kind=kind)
    out, (Wc, _), (Wl, bl) = _fwd(d, G=8)
    ref = O.linear_forward_full(*(d[k].double() for k in ("ln_w", "ln_b", "W1", "b1", "XQ", "XV", "XK", "eta")), G=8)
    assert out.dtype == dt
    assert rel_l2(out, ref["out"]) <= BF16_RTOL
    assert rel_l2(Wl, ref["W1_last"]) <= BF16_RTOL
    assert rel_l2(Wc, ref["W1_ckpt"]) <= BF16_RTOL


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("NC,G,F_", [(1, 1, 64), (2, 1, 64), (3, 2, 32), (5, 5, 64), (2, 2, 32), (7, 3, 64)])
def test_linear_fwd_16bit_edges(dt, NC, G, F_):
    """16-bit activations run the row-split kernel, whose state update enters
    the next mini-batch as a look-ahead correction: one and two mini-batches,
    groups that do and do not divide NC, F = 32.  Outputs and states against
    the fp64 oracle (rel-L2 <= 2e-2); the saved slot against the relations it
    must satisfy (fp32 rounding, 1e-4 of the magnitudes, where the kernel forms
    the value in fp32; the state through the bf16 update operands, 2e-2)."""
    _say("linear fwd 16-bit edges", dt, f"NC{NC} G{G} F{F_}")
    B, H = 2, 2
    d = O.make_inputs(B, H, NC, 16, F_, seed=30 + NC + F_, dtype=dt, eta_kind="causal")
    gen = torch.Generator().manual_seed(31)
    d["ln_w"] = 1 + 0.2 * torch.randn(H, F_, generator=gen)
    d["ln_b"] = 0.2 * torch.randn(H, F_, generator=gen)
    d["b1"] = 0.1 * torch.randn(B, H, 1, F_, generator=gen)
    out, (Wc, bc), (Wl, bl), saved = _fwd(d, G=G, want_saved=True)
    torch.cuda.synchronize()
    ref = O.linear_forward_full(*(d[k].double() for k in ("ln_w", "ln_b", "W1", "b1", "XQ", "XV", "XK", "eta")), G=G)
    for name, mine in (("out", out), ("W1_last", Wl), ("b1_last", bl), ("W1_ckpt", Wc), ("b1_ckpt", bc)):
        err = rel_l2(mine, ref[name])
        _say(f"  {name}: rel-L2 {err:.3e}")
        assert err <= BF16_RTOL, name
    sv = {k: v.cpu().double() for k, v in _unpack_saved(saved, B, H, NC, F_).items()}
    XK, XV, XQ = d["XK"].double(), d["XV"].double(), d["XQ"].double()
    e = d["eta"].double()[..., -1, :]
    dW = torch.einsum("bhstf,bhst,bhsto->bhfo", XK, e, sv["G"])
    assert rel_l2(Wl, d["W1"].double() - dW) <= BF16_RTOL
    db = torch.einsum("bhst,bhsto->bho", e, sv["G"]).unsqueeze(2)
    assert max_abs(bl, d["b1"].double() - db) <= 1e-4 * (1 + db.abs().max().item())
    lw, lb = d["ln_w"].double()[None, :, None, None, :], d["ln_b"].double()[None, :, None, None, :]
    xh = sv["XH"]
    gx = (lw * xh + lb - (XV - XK)) * lw
    Gr = (gx - gx.mean(-1, keepdim=True) - xh * sv["CC"][..., None]) * sv["RSTD"][..., None]
    assert max_abs(Gr, sv["G"]) <= 1e-4 * (1 + sv["G"].abs().max().item())
    assert max_abs(sv["CC"], (gx * xh).mean(-1)) <= 1e-4 * (1 + sv["CC"].abs().max().item())
    assert max_abs(xh.mean(-1), torch.zeros_like(sv["RSTD"])) <= 1e-4
    assert rel_l2(out, XQ + lw * sv["XHB"] + lb) <= 1e-2
    assert bool((sv["RSB"] > 0).all()) and bool((sv["RSTD"] > 0).all())


def test_linear_fwd_deterministic():
    _say("linear fwd determinism")
    d = O.make_inputs(2, 2, 8, 16, 64, seed=2, dtype=torch.bfloat16)
    a, _, _ = _fwd(d, G=4)
    b, _, _ = _fwd(d, G=4)
    assert torch.equal(a, b)


def _bwd(d, dout, G):
    from ttt_amd.linear import linear_backward
    g = to_dev(d)
    _, (Wc, _), (Wl, _), saved = _fwd(d, G, want_saved=True)
    (dlw, dlb, dW, db), (dxq, dxv, dxk, deta) = linear_backward(
        g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], Wc, Wl, saved, dout.cuda(), G)
    return dict(dXQ=dxq, dXV=dxv, dXK=dxk, deta=deta, dW1=dW, db1=db, dln_w=dlw, dln_b=dlb)


@pytest.mark.parametrize("kind", ["causal", "layer"])
def test_linear_bwd_fp32(kind):
    _say("linear bwd fp32", kind)
    d = O.make_inputs(2, 2, 6, 16, 64, seed=4, dtype=torch.float32, eta_kind=kind, with_grad=True)
    gen = torch.Generator().manual_seed(10)
    d["ln_w"] = 1 + 0.2 * torch.randn(2, 64, generator=gen)
    d["ln_b"] = 0.2 * torch.randn(2, 64, generator=gen)
    mine = _bwd(d, d["dOut"], G=4)
    ref = oracle_linear_grads(d, d["dOut"], G=0)
    ref32 = oracle_linear_grads(d, d["dOut"], G=0, dtype=torch.float32)
    bad = []
    for k in mine:
        err, bound = max_abs(mine[k], ref[k]), fp32_bound(ref[k], ref32[k])
        _say(f"  {k}: max-abs {err:.3e} (fp32 oracle {max_abs(ref32[k], ref[k]):.3e}, bound {bound:.3e})"
             f"  rel-L2 {rel_l2(mine[k], ref[k]):.3e}")
        if err > bound:
            bad.append(k)
    assert not bad


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("F_,NC,G", [(64, 24, 8), (32, 9, 4)], ids=["F64", "F32"])
def test_linear_bwd_16bit(dt, F_, NC, G):
    """16-bit activations at both widths (F = 32: two feature tiles per
    handoff frag set; a group size that does not divide NC)"""
    _say("linear bwd", dt, f"F{F_} NC{NC} G{G}")
    d = eta_own_dtype(O.make_inputs(2, 3, NC, 16, F_, seed=6, dtype=dt, with_grad=True), dt)
    mine = _bwd(d, d["dOut"], G=G)
    ref = oracle_linear_grads(d, d["dOut"], G=0)
    bad = []
    for k in mine:
        err = rel_l2(mine[k], ref[k])
        _say(f"  {k}: rel-L2 {err:.3e}")
        if err > BF16_RTOL:
            bad.append(k)
    assert not bad


@pytest.mark.parametrize("NC,G,F_", [(1, 1, 64), (7, 3, 64), (5, 5, 32), (9, 4, 32)])
def test_linear_bwd_edges_fp32(NC, G, F_):
    """single mini-batch, a group size that does not divide NC, F = 32"""
    _say(f"linear bwd fp32 NC{NC} G{G} F{F_}")
    d = O.make_inputs(1, 2, NC, 16, F_, seed=20 + NC, dtype=torch.float32, with_grad=True)
    mine = _bwd(d, d["dOut"], G=G)
    ref = oracle_linear_grads(d, d["dOut"], G=0)
    ref32 = oracle_linear_grads(d, d["dOut"], G=0, dtype=torch.float32)
    bad = []
    for k in mine:
        err, bound = max_abs(mine[k], ref[k]), fp32_bound(ref[k], ref32[k])
        _say(f"  {k}: max-abs {err:.3e} bound {bound:.3e}")
        if err > bound:
            bad.append(k)
    assert not bad
