"""Pins the CPU oracle (oracle/ttt_oracle.py) to library routines, closed
forms, brute force and invariants.  The reference ships no tests or golden
vectors for this path, so these checks are what fixes the oracle: each one is
chosen so that a plausible slip (dropped term, wrong sign, transposed operand,
wrong eta row, wrong eps) fails it."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ttt_oracle as O

DT = torch.float64


def _rand(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=DT) * scale


# --- math helpers -----------------------------------------------------------

def test_ln_fwd_matches_layer_norm():
    x = _rand(3, 5, 64, seed=1) * 3 + 0.7
    g = _rand(64, seed=2)
    b = _rand(64, seed=3)
    ref = F.layer_norm(x, (64,), g, b, eps=1e-8)
    torch.testing.assert_close(O.ln_fwd(x, g, b), ref, rtol=0, atol=1e-12)


def test_ln_fused_l2_bwd_is_gradient_of_l2_of_layer_norm():
    x = _rand(4, 16, 64, seed=4, scale=2.0).requires_grad_(True)
    t = _rand(4, 16, 64, seed=5)
    g = _rand(64, seed=6)
    b = _rand(64, seed=7)
    loss = 0.5 * ((F.layer_norm(x, (64,), g, b, eps=1e-8) - t) ** 2).sum()
    (ref,) = torch.autograd.grad(loss, x)
    torch.testing.assert_close(O.ln_fused_l2_bwd(x.detach(), t, g, b), ref, rtol=0, atol=1e-11)


def test_ln_eps_is_1e8():
    # a near-constant row makes eps visible: 1e-6 would change the result
    x = torch.full((1, 64), 2.0, dtype=DT)
    x[0, 0] += 1e-4
    g = torch.ones(64, dtype=DT)
    b = torch.zeros(64, dtype=DT)
    ref8 = F.layer_norm(x, (64,), g, b, eps=1e-8)
    ref6 = F.layer_norm(x, (64,), g, b, eps=1e-6)
    assert (ref8 - ref6).abs().max() > 1e-3
    torch.testing.assert_close(O.ln_fwd(x, g, b), ref8, rtol=0, atol=1e-10)


def test_gelu_bwd_is_gelu_tanh_derivative():
    x = torch.linspace(-8, 8, 2001, dtype=DT).requires_grad_(True)
    (ref,) = torch.autograd.grad(F.gelu(x, approximate="tanh").sum(), x)
    # the ops path's rounded constants (0.79788456, 0.1070322243) differ from
    # sqrt(2/pi) at the 1e-9 level
    assert (O.gelu_bwd(x.detach()) - ref).abs().max() < 5e-8


# --- one mini-batch -----------------------------------------------------------

def _brute_linear(W, b, XQ, XK, XV, eta, lnw, lnb):
    """Per-token primal statement of the dual form: token i reads out with
    W_i = W - sum_j eta[i,j] xk_j^T g_j and b_i = b - sum_j eta[i,j] g_j."""
    B, H, K, Fd = XQ.shape
    out = torch.empty_like(XQ)
    for bb in range(B):
        for h in range(H):
            Z1 = XK[bb, h] @ W[bb, h] + b[bb, h]
            gr = O.ln_fused_l2_bwd(Z1, XV[bb, h] - XK[bb, h], lnw[h], lnb[h])
            for i in range(K):
                Wi = W[bb, h].clone()
                bi = b[bb, h, 0].clone()
                for j in range(K):
                    Wi -= eta[bb, h, i, j] * torch.outer(XK[bb, h, j], gr[j])
                    bi -= eta[bb, h, i, j] * gr[j]
                z = XQ[bb, h, i] @ Wi + bi
                out[bb, h, i] = XQ[bb, h, i] + O.ln_fwd(z, lnw[h], lnb[h])
    return out


def _step_inputs(B=2, H=2, K=16, Fd=64, FF=0, seed=0, eta_kind="causal"):
    d = O.make_inputs(B, H, 1, K, Fd, FF=FF, seed=seed, dtype=DT, eta_kind=eta_kind)
    d = {k: v.to(DT) for k, v in d.items()}
    d["ln_w"] = 1.0 + 0.1 * _rand(H, Fd, seed=seed + 11)
    d["ln_b"] = 0.1 * _rand(H, Fd, seed=seed + 12)
    d["b1"] = 0.05 * _rand(*d["b1"].shape, seed=seed + 13)
    if FF:
        d["b2"] = 0.05 * _rand(*d["b2"].shape, seed=seed + 14)
    xs = {k: d[k][:, :, 0] for k in ("XQ", "XK", "XV", "eta")}
    return d, xs


def test_linear_dual_form_matches_brute_force_causal_eta():
    d, xs = _step_inputs(eta_kind="causal")
    p = {"W1_states": d["W1"], "b1_states": d["b1"], "ttt_norm_weight": d["ln_w"], "ttt_norm_bias": d["ln_b"]}
    _, out = O.linear_mini_batch(p, xs)
    ref = _brute_linear(d["W1"], d["b1"], xs["XQ"], xs["XK"], xs["XV"], xs["eta"], d["ln_w"], d["ln_b"])
    torch.testing.assert_close(out, ref, rtol=0, atol=1e-10)


def test_linear_final_state_closed_form():
    d, xs = _step_inputs(eta_kind="causal", seed=3)
    p = {"W1_states": d["W1"], "b1_states": d["b1"], "ttt_norm_weight": d["ln_w"], "ttt_norm_bias": d["ln_b"]}
    new, _ = O.linear_mini_batch(p, xs)
    W, b = d["W1"], d["b1"]
    Z1 = xs["XK"] @ W + b
    gr = O.ln_fused_l2_bwd(Z1, xs["XV"] - xs["XK"], d["ln_w"][:, None], d["ln_b"][:, None])
    e = xs["eta"][:, :, -1]  # last row
    W_ref = W - torch.einsum("bhk,bhkf,bhkg->bhfg", e, xs["XK"], gr)
    b_ref = b - torch.einsum("bhk,bhkg->bhg", e, gr)[:, :, None]
    torch.testing.assert_close(new["W1_states"], W_ref, rtol=0, atol=1e-12)
    torch.testing.assert_close(new["b1_states"], b_ref, rtol=0, atol=1e-12)


@pytest.mark.parametrize("kind", ["layer", "tokens"])
def test_linear_row_constant_eta_equals_primal(kind):
    d, xs = _step_inputs(eta_kind=kind, seed=5)
    p = {"W1_states": d["W1"], "b1_states": d["b1"], "ttt_norm_weight": d["ln_w"], "ttt_norm_bias": d["ln_b"]}
    new, out = O.linear_mini_batch(p, xs)
    z = xs["XQ"] @ new["W1_states"] + new["b1_states"]
    ref = xs["XQ"] + O.ln_fwd(z, d["ln_w"][:, None], d["ln_b"][:, None])
    torch.testing.assert_close(out, ref, rtol=0, atol=1e-11)


def _brute_mlp(d, xs):
    W1, b1, W2, b2 = d["W1"], d["b1"], d["W2"], d["b2"]
    XQ, XK, XV, eta = xs["XQ"], xs["XK"], xs["XV"], xs["eta"]
    B, H, K, Fd = XQ.shape
    out = torch.empty_like(XQ)
    for bb in range(B):
        for h in range(H):
            lw, lb = d["ln_w"][h], d["ln_b"][h]
            Z1 = XK[bb, h] @ W1[bb, h] + b1[bb, h]
            X2 = F.gelu(Z1, approximate="tanh")
            Z2 = X2 @ W2[bb, h] + b2[bb, h]
            g2 = O.ln_fused_l2_bwd(Z2, XV[bb, h] - XK[bb, h], lw, lb)
            g1 = (g2 @ W2[bb, h].T) * O.gelu_bwd(Z1)
            for i in range(K):
                W1i = W1[bb, h] - sum(eta[bb, h, i, j] * torch.outer(XK[bb, h, j], g1[j]) for j in range(K))
                b1i = b1[bb, h, 0] - sum(eta[bb, h, i, j] * g1[j] for j in range(K))
                x2b = F.gelu(XQ[bb, h, i] @ W1i + b1i, approximate="tanh")
                W2i = W2[bb, h] - sum(eta[bb, h, i, j] * torch.outer(X2[j], g2[j]) for j in range(K))
                b2i = b2[bb, h, 0] - sum(eta[bb, h, i, j] * g2[j] for j in range(K))
                out[bb, h, i] = XQ[bb, h, i] + O.ln_fwd(x2b @ W2i + b2i, lw, lb)
    return out


def test_mlp_dual_form_matches_brute_force_causal_eta():
    d, xs = _step_inputs(B=1, H=2, FF=128, eta_kind="causal", seed=7)
    p = {"W1_states": d["W1"], "b1_states": d["b1"], "W2_states": d["W2"], "b2_states": d["b2"],
         "ttt_norm_weight": d["ln_w"], "ttt_norm_bias": d["ln_b"]}
    _, out = O.mlp_mini_batch(p, xs)
    torch.testing.assert_close(out, _brute_mlp(d, xs), rtol=0, atol=1e-10)


def test_mlp_row_constant_eta_equals_primal_and_closed_form_state():
    d, xs = _step_inputs(B=1, H=2, FF=256, eta_kind="layer", seed=9)
    p = {"W1_states": d["W1"], "b1_states": d["b1"], "W2_states": d["W2"], "b2_states": d["b2"],
         "ttt_norm_weight": d["ln_w"], "ttt_norm_bias": d["ln_b"]}
    new, out = O.mlp_mini_batch(p, xs)
    lw, lb = d["ln_w"][:, None], d["ln_b"][:, None]
    x2b = F.gelu(xs["XQ"] @ new["W1_states"] + new["b1_states"], approximate="tanh")
    ref = xs["XQ"] + O.ln_fwd(x2b @ new["W2_states"] + new["b2_states"], lw, lb)
    torch.testing.assert_close(out, ref, rtol=0, atol=1e-11)
    # closed form of the update with the last eta row
    Z1 = xs["XK"] @ d["W1"] + d["b1"]
    X2 = F.gelu(Z1, approximate="tanh")
    g2 = O.ln_fused_l2_bwd(X2 @ d["W2"] + d["b2"], xs["XV"] - xs["XK"], lw, lb)
    g1 = (g2 @ d["W2"].transpose(-1, -2)) * O.gelu_bwd(Z1)
    e = xs["eta"][:, :, -1]
    torch.testing.assert_close(new["W1_states"], d["W1"] - torch.einsum("bhk,bhkf,bhkg->bhfg", e, xs["XK"], g1), rtol=0, atol=1e-12)
    torch.testing.assert_close(new["W2_states"], d["W2"] - torch.einsum("bhk,bhkf,bhkg->bhfg", e, X2, g2), rtol=0, atol=1e-12)


# --- scan, side outputs -------------------------------------------------------

def _seq(B=1, H=2, NC=6, FF=0, seed=0, kind="causal"):
    d = O.make_inputs(B, H, NC, 16, 64, FF=FF, seed=seed, dtype=DT, eta_kind=kind)
    return {k: v.to(DT) for k, v in d.items()}


@pytest.mark.parametrize("G", [0, 1, 4, 6])
def test_scan_forward_invariant_to_checkpoint_group(G):
    d = _seq(seed=1)
    args = (d["XK"], d["XQ"], d["XV"], d["eta"], d["ln_w"], d["ln_b"], d["W1"], d["b1"])
    ref = O.ttt_linear(*args, 0)
    torch.testing.assert_close(O.ttt_linear(*args, G), ref, rtol=0, atol=0)
    assert ref.shape == (1, 6, 16, 2, 64)  # [B,NC,K,H,F]


def test_linear_side_outputs_are_states_of_step_loop():
    d = _seq(seed=2)
    full = O.linear_forward_full(d["ln_w"], d["ln_b"], d["W1"], d["b1"], d["XQ"], d["XV"], d["XK"], d["eta"], G=4)
    out_ops, carry = O.ttt_linear(d["XK"], d["XQ"], d["XV"], d["eta"], d["ln_w"], d["ln_b"], d["W1"], d["b1"], 2,
                                  return_state=True)
    torch.testing.assert_close(full["out"], out_ops.permute(0, 3, 1, 2, 4), rtol=0, atol=0)
    torch.testing.assert_close(full["W1_last"], carry["W1_states"], rtol=0, atol=0)
    assert full["W1_ckpt"].shape == (1, 2, 2, 64, 64)
    torch.testing.assert_close(full["W1_ckpt"][:, :, 0], d["W1"], rtol=0, atol=0)
    # checkpoint 1 = state entering mini-batch 4 = carry after running 4 steps
    sub = {k: d[k][:, :, :4] for k in ("XK", "XQ", "XV", "eta")}
    _, c4 = O.ttt_linear(sub["XK"], sub["XQ"], sub["XV"], sub["eta"], d["ln_w"], d["ln_b"], d["W1"], d["b1"], 0,
                         return_state=True)
    torch.testing.assert_close(full["W1_ckpt"][:, :, 1], c4["W1_states"], rtol=0, atol=0)
    torch.testing.assert_close(full["b1_ckpt"][:, :, 1], c4["b1_states"], rtol=0, atol=0)


def test_mlp_memo_is_state_after_step_s_times_M():
    d = _seq(FF=64, NC=5, seed=3)
    full = O.mlp_forward_full(d["ln_w"], d["ln_b"], d["W1"], d["b1"], d["W2"], d["b2"], d["XQ"], d["XV"], d["XK"],
                              d["eta"], G=2, M=2)
    assert full["W1_memo"].shape[2] == 3  # ceil(5/2)
    for s, step in enumerate(range(0, 5, 2)):
        sub = {k: d[k][:, :, : step + 1] for k in ("XK", "XQ", "XV", "eta")}
        _, c = O.ttt_mlp(sub["XK"], sub["XQ"], sub["XV"], sub["eta"], d["ln_w"], d["ln_b"], d["W1"], d["b1"],
                         d["W2"], d["b2"], 0, return_state=True)
        torch.testing.assert_close(full["W2_memo"][:, :, s], c["W2_states"], rtol=0, atol=0)
        torch.testing.assert_close(full["b1_memo"][:, :, s], c["b1_states"], rtol=0, atol=0)


def test_cached_readout_equals_mini_batch_with_zero_eta():
    d = _seq(FF=128, NC=1, seed=4)
    d["b1"] = 0.1 * _rand(*d["b1"].shape, seed=40)
    d["b2"] = 0.1 * _rand(*d["b2"].shape, seed=41)
    d["ln_w"] = 1 + 0.1 * _rand(2, 64, seed=42)
    xs = {k: d[k][:, :, 0] for k in ("XQ", "XK", "XV")}
    xs["eta"] = torch.zeros(1, 2, 16, 16, dtype=DT)
    p = {"W1_states": d["W1"], "b1_states": d["b1"], "W2_states": d["W2"], "b2_states": d["b2"],
         "ttt_norm_weight": d["ln_w"], "ttt_norm_bias": d["ln_b"]}
    _, ref = O.mlp_mini_batch(p, xs)
    out = O.cached_readout(d["XQ"], d["W1"], d["b1"], d["W2"], d["b2"], d["ln_w"], d["ln_b"], eps=1e-8)
    torch.testing.assert_close(out[:, :, 0].to(DT), ref, rtol=0, atol=1e-6)


def test_cached_readout_uses_each_chain_weights():
    # the reference kernel reads only chain (0,0); the oracle must not
    d = _seq(B=2, FF=64, NC=2, seed=5)
    W1 = d["W1"].clone()
    W1[1, 1] *= 3.0
    o1 = O.cached_readout(d["XQ"], W1, d["b1"], d["W2"], d["b2"], d["ln_w"], d["ln_b"])
    o0 = O.cached_readout(d["XQ"], d["W1"], d["b1"], d["W2"], d["b2"], d["ln_w"], d["ln_b"])
    assert (o1[1, 1] - o0[1, 1]).abs().max() > 1e-3
    torch.testing.assert_close(o1[0], o0[0], rtol=0, atol=0)


# --- memo combiner (ttt_layer.py:506-561) -------------------------------------------

def _memo_inputs(B=1, H=2, NC=6, M=2, F_=16, FF=32, seed=50):
    g = torch.Generator().manual_seed(seed)
    NS = O.ceil_div(NC, M)
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(DT)
    return dict(XQ=r(B, H, NC, 16, F_), XK=r(B, H, NC, 16, F_), XU=r(B, H, NC, 16, F_, sc=0.3),
                XQW=r(B, H, NC, 16, F_), W1=r(B, H, NS, F_, FF, sc=0.2), b1=r(B, H, NS, 1, FF, sc=0.1),
                W2=r(B, H, NS, FF, F_, sc=0.2), b2=r(B, H, NS, 1, F_, sc=0.1),
                ln_w=1 + r(H, F_, sc=0.1), ln_b=r(H, F_, sc=0.1)), M


def _combine(d, M):
    return O.memo_combine(d["XQ"], d["XK"], d["XU"], d["XQW"], d["W1"], d["b1"], d["W2"], d["b2"],
                          d["ln_w"], d["ln_b"], M)


def test_memo_combine_one_segment_is_identity():
    d, _ = _memo_inputs(NC=3, M=3)
    torch.testing.assert_close(_combine(d, 3), d["XQW"], rtol=0, atol=0)


def test_memo_combine_zero_gate_input_averages_uniformly():
    """XU = 0: every gate is 1/(i+1), so a token of segment i gets the plain mean
    of XQW and the readouts of memo states 0..i-1 (each state distinct, so a
    wrong state index or range fails)."""
    d, M = _memo_inputs(NC=7, M=2)
    d["XU"] = torch.zeros_like(d["XU"])
    out = _combine(d, M)
    NC = d["XQ"].shape[2]
    for s in range(NC):
        i = s // M
        q = d["XQ"][:, :, s:s + 1]
        tot = d["XQW"][:, :, s:s + 1].clone()
        for j in range(i):
            tot = tot + O.cached_readout(q, d["W1"][:, :, j], d["b1"][:, :, j], d["W2"][:, :, j], d["b2"][:, :, j],
                                         d["ln_w"], d["ln_b"], dtype=DT)
        torch.testing.assert_close(out[:, :, s:s + 1], tot / (i + 1), rtol=0, atol=1e-12)


def test_memo_combine_is_a_convex_combination():
    """Identical memo states and XQW equal to their readout: any gates give back XQW."""
    d, M = _memo_inputs(NC=6, M=2, seed=51)
    for k in ("W1", "b1", "W2", "b2"):
        d[k] = d[k][:, :, :1].expand_as(d[k]).contiguous()
    d["XQW"] = O.cached_readout(d["XQ"], d["W1"][:, :, 0], d["b1"][:, :, 0], d["W2"][:, :, 0], d["b2"][:, :, 0],
                                d["ln_w"], d["ln_b"], dtype=DT)
    d["XU"] = d["XU"] * 5  # far from uniform gates
    torch.testing.assert_close(_combine(d, M), d["XQW"], rtol=0, atol=1e-12)


def test_memo_combine_gates_of_one_token_by_hand():
    """The gates of one token recomputed from scalar loops (summary = mean of XK
    over the segment's tokens, sims = dot products, softmax = exp / sum)."""
    d, M = _memo_inputs(NC=6, M=2, seed=52)
    d["XU"] = d["XU"] * 3
    b, h, s, t = 0, 1, 5, 7  # segment 2
    i = s // M
    F_ = d["XQ"].shape[-1]
    summ = []
    for j in range(i + 1):
        acc = [0.0] * F_
        toks = [(ss, tt) for ss in range(j * M, (j + 1) * M) for tt in range(16)]
        for ss, tt in toks:
            for f in range(F_):
                acc[f] += float(d["XK"][b, h, ss, tt, f])
        summ.append([a / len(toks) for a in acc])
    sims = [sum(float(d["XU"][b, h, s, t, f]) * summ[j][f] for f in range(F_)) for j in range(i + 1)]
    e = [math.exp(x - max(sims)) for x in sims]
    gam = [x / sum(e) for x in e]
    q = d["XQ"][b:b + 1, h:h + 1, s:s + 1, t:t + 1]
    ref = gam[i] * d["XQW"][b, h, s, t]
    for j in range(i):
        r = O.cached_readout(q, d["W1"][b:b + 1, h:h + 1, j], d["b1"][b:b + 1, h:h + 1, j], d["W2"][b:b + 1, h:h + 1, j],
                             d["b2"][b:b + 1, h:h + 1, j], d["ln_w"][h:h + 1], d["ln_b"][h:h + 1], dtype=DT)
        ref = ref + gam[j] * r[0, 0, 0, 0]
    torch.testing.assert_close(_combine(d, M)[b, h, s, t], ref, rtol=0, atol=1e-12)


def test_memo_combine_gradients_match_finite_differences():
    d, M = _memo_inputs(NC=5, M=2, F_=8, FF=16, seed=53)
    XU = d["XU"].clone().requires_grad_(True)
    XQW = d["XQW"].clone().requires_grad_(True)

    def f(xu, xqw):
        return O.memo_combine(d["XQ"], d["XK"], xu, xqw, d["W1"], d["b1"], d["W2"], d["b2"], d["ln_w"], d["ln_b"], M)
    assert torch.autograd.gradcheck(f, (XU, XQW), eps=1e-6, atol=1e-6, rtol=1e-5)


def test_memo_combine_xk_gradient_is_through_the_current_summary_only():
    """The reference differentiates segment i's summary only where it is the
    current one (ttt_layer.py:519,528; the cached copy is detached, :521,559).
    XK of segment i moves the outputs of segments i..NS-1, so its reference
    gradient is the finite-difference derivative of segment i's outputs alone;
    segment 0's summary is never differentiated."""
    d, M = _memo_inputs(NC=7, M=2, F_=8, FF=16, seed=54)
    d["XU"] = d["XU"] * 3
    XK = d["XK"].clone().requires_grad_(True)
    w = torch.randn(d["XQ"].shape, generator=torch.Generator().manual_seed(55), dtype=DT)
    out = O.memo_combine(d["XQ"], XK, d["XU"], d["XQW"], d["W1"], d["b1"], d["W2"], d["b2"], d["ln_w"], d["ln_b"], M)
    (out * w).sum().backward()
    NC = d["XQ"].shape[2]
    assert float(XK.grad[:, :, :M].abs().max()) == 0.0
    v = torch.randn(d["XK"].shape, generator=torch.Generator().manual_seed(56), dtype=DT)
    h = 1e-6
    for i in range(1, O.ceil_div(NC, M)):
        s0, s1 = i * M, min((i + 1) * M, NC)
        vi = torch.zeros_like(v)
        vi[:, :, s0:s1] = v[:, :, s0:s1]

        def seg_loss(xk):
            o = O.memo_combine(d["XQ"], xk, d["XU"], d["XQW"], d["W1"], d["b1"], d["W2"], d["b2"], d["ln_w"],
                               d["ln_b"], M)
            return float((o[:, :, s0:s1] * w[:, :, s0:s1]).sum())
        fd = (seg_loss(d["XK"] + h * vi) - seg_loss(d["XK"] - h * vi)) / (2 * h)
        ad = float((XK.grad * vi).sum())
        assert abs(fd - ad) <= 1e-6 * max(1.0, abs(fd)), (i, fd, ad)
        # every token of the segment gets the same gradient (a mean's derivative)
        gseg = XK.grad[:, :, s0:s1]
        torch.testing.assert_close(gseg, gseg[:, :, :1, :1].expand_as(gseg), rtol=0, atol=1e-14)


# --- backward -------------------------------------------------------------------

def test_linear_backward_autograd_matches_finite_differences():
    d = O.make_inputs(1, 1, 2, 4, 8, seed=6, dtype=DT)
    d = {k: v.to(DT) for k, v in d.items()}
    d["W1"] = d["W1"] * 10
    names = ["XK", "XQ", "XV", "eta", "ln_w", "ln_b", "W1", "b1"]
    args = [d[n].clone().requires_grad_(True) for n in names]

    def f(*a):
        return O.ttt_linear(*a, 1)
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-5, rtol=1e-4)


def test_mlp_backward_autograd_matches_finite_differences():
    d = O.make_inputs(1, 1, 2, 4, 8, FF=16, seed=7, dtype=DT)
    d = {k: v.to(DT) for k, v in d.items()}
    d["W1"] = d["W1"] * 10
    d["W2"] = d["W2"] * 10
    names = ["XK", "XQ", "XV", "eta", "ln_w", "ln_b", "W1", "b1", "W2", "b2"]
    args = [d[n].clone().requires_grad_(True) for n in names]

    def f(*a):
        return O.ttt_mlp(*a, 1)
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-5, rtol=1e-4)


def test_eta_builders():
    u = _rand(1, 1, 1, 16, seed=8)
    lr = torch.sigmoid(u) / 64
    causal = O.make_eta(u, 64, "causal")[0, 0, 0]
    assert torch.all(torch.triu(causal, 1) == 0)
    torch.testing.assert_close(torch.diagonal(causal), lr[0, 0, 0] / torch.arange(1, 17, dtype=DT))
    layer = O.make_eta(u, 64, "layer")[0, 0, 0]
    torch.testing.assert_close(layer, (lr[0, 0, 0] / 16).expand(16, 16))
