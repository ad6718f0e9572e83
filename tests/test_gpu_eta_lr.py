"""eta given as learning rates lr [B,H,NC,K] and expanded on chip (ttt_eta.h),
against (1) the dense path fed the same eta, built in fp32 from lr the way the
oracle builds it (bit-identical eta values, so every output and every input
gradient must be bitwise equal, and dlr must equal the row sums of the dense
deta times d eta / d lr), and (2) the oracle's autograd with lr as the leaf
(ttt_layer.py:151-163,309 for the layer rule).  Tolerances: fp32 max-abs
1e-4, or C_FP32 = 8 times the fp32 oracle's own error against fp64 where
that is larger (tests/_util.fp32_bound); bf16 rel-L2 2e-2."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import fp32_bound, max_abs, rel_l2, to_dev

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _inputs(B, H, NC, F_, FF, dt, rule, seed, K=16):
    """Inputs with lr = sigmoid(u)/F drawn as the oracle draws them, and the
    dense eta the oracle's make_eta builds from the same lr in fp32."""
    d = O.make_inputs(B, H, NC, K, F_, FF=FF, seed=seed, dtype=dt, with_grad=True, eta_kind=rule)
    gen = torch.Generator().manual_seed(seed + 1000)
    u = torch.randn(B, H, NC, K, generator=gen)
    d["lr"] = torch.sigmoid(u) / F_
    d["eta32"] = O.eta_from_lr(d["lr"], rule)  # fp32, from the same lr
    gen = torch.Generator().manual_seed(seed + 2000)
    d["ln_w"] = 1 + 0.2 * torch.randn(H, F_, generator=gen)
    d["ln_b"] = 0.2 * torch.randn(H, F_, generator=gen)
    return d


def _coef(rule, K=16):
    i = torch.arange(K, dtype=torch.float64)
    if rule == "layer":
        return torch.full((K, K), 1.0 / K, dtype=torch.float64)
    return torch.tril(torch.ones(K, K, dtype=torch.float64)) / (i + 1)[:, None]


def _oracle(kind, d, G, rule, dtype=torch.float64):
    names = ["XK", "XQ", "XV", "ln_w", "ln_b", "W1", "b1"] + (["W2", "b2"] if kind == "mlp" else [])
    a = {n: d[n].detach().cpu().to(dtype).requires_grad_(True) for n in names}
    lr = d["lr"].to(dtype).requires_grad_(True)
    eta = O.eta_from_lr(lr, rule)
    if kind == "mlp":
        out = O.ttt_mlp(a["XK"], a["XQ"], a["XV"], eta, a["ln_w"], a["ln_b"], a["W1"], a["b1"], a["W2"], a["b2"], G)
    else:
        out = O.ttt_linear(a["XK"], a["XQ"], a["XV"], eta, a["ln_w"], a["ln_b"], a["W1"], a["b1"], G)
    out.backward(d["dOut"].to(dtype).permute(0, 2, 3, 1, 4))
    res = {"out": out.detach().permute(0, 3, 1, 2, 4), "dlr": lr.grad}
    res.update({"d" + n: a[n].grad for n in names})
    return res


def _run(kind, d, G, rule, eta_key):
    """(out, grads) of the HIP path through the autograd Function, with eta
    either dense (eta_key 'eta32' cast to the activation dtype, 'eta32_f32'
    kept in fp32) or lr."""
    from ttt_amd.linear import TTTLinearFunction
    from ttt_amd.mlp import TTTMLPFunction
    g = to_dev(d)
    dt = d["XQ"].dtype
    names = ["ln_w", "ln_b", "W1", "b1"] + (["W2", "b2"] if kind == "mlp" else []) + ["XQ", "XV", "XK"]
    leaf = {n: g[n].clone().requires_grad_(True) for n in names}
    if eta_key == "lr":
        eta = g["lr"].clone().requires_grad_(True)
        extra = ("layer",) if rule == "layer" else ("causal",)
    elif eta_key == "eta32_f32":
        eta = g["eta32"].clone().requires_grad_(True)
        extra = ("dense",)
    else:
        eta = g[eta_key].to(dt).clone().requires_grad_(True)
        extra = ("dense",)
    if kind == "mlp":
        out = TTTMLPFunction.apply(*(leaf[n] for n in names), eta, G, 0, O.LN_EPS, *extra)[0]
    else:
        out = TTTLinearFunction.apply(*(leaf[n] for n in names), eta, G, O.LN_EPS, *extra)
    out.backward(g["dOut"])
    torch.cuda.synchronize()
    grads = {"d" + n: leaf[n].grad for n in names}
    grads["deta"] = eta.grad
    return out.detach(), grads


@pytest.mark.parametrize("kind", ["linear", "mlp"])
@pytest.mark.parametrize("rule", ["layer", "causal"])
def test_lr_fp32_bitwise_equals_dense(kind, rule):
    """fp32 activations: the lr path and the dense path see identical eta
    values, so outputs and input gradients agree bit for bit; dlr is the
    coefficient-weighted row sum of the dense path's deta."""
    _say(f"{kind} lr vs dense fp32, {rule}")
    B, H, NC, F_, FF = 2, 2, 6, 64, (128 if kind == "mlp" else 0)
    d = _inputs(B, H, NC, F_, FF, torch.float32, rule, seed=71)
    out_l, g_l = _run(kind, d, 4, rule, "lr")
    out_d, g_d = _run(kind, d, 4, rule, "eta32")
    assert torch.equal(out_l, out_d)
    for k in g_l:
        if k != "deta":
            assert torch.equal(g_l[k], g_d[k]), k
    dlr_ref = (g_d["deta"].double().cpu() * _coef(rule)).sum(-2)
    err = max_abs(g_l["deta"], dlr_ref)
    _say(f"  dlr vs rows of dense deta: max-abs {err:.3e}")
    assert err <= 1e-6 * max(1.0, float(dlr_ref.abs().max()))


# (kind, K, F, FF): the specialised kernels (K = 16, F = 64), the
# register-resident ones (K = 64, F = FF = 32) and the staged general-shape
# ones (K = 32, F = 128)
DENSE_F32_SHAPES = [("linear", 16, 64, 0), ("mlp", 16, 64, 256), ("linear", 64, 32, 0), ("mlp", 64, 32, 32),
                    ("linear", 32, 128, 0), ("mlp", 32, 128, 128)]


@pytest.mark.parametrize("kind,K,F_,FF", DENSE_F32_SHAPES)
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_lr_16bit_bitwise_equals_dense_fp32_eta(kind, K, F_, FF, dt):
    """16-bit activations with a dense eta kept in fp32 (TTT_ETA_DENSE_F32):
    the kernels read the same fp32 eta values the lr rule forms on chip, so
    outputs and input gradients agree bit for bit with the lr path; deta
    comes back in fp32 and its coefficient-weighted row sums are dlr."""
    rule = "causal"
    _say(f"{kind} K{K} F{F_} FF{FF} {dt}: lr vs dense fp32 eta")
    B, H, NC = 2, 2, 5
    d = _inputs(B, H, NC, F_, FF, dt, rule, seed=77, K=K)
    out_l, g_l = _run(kind, d, 2, rule, "lr")
    out_d, g_d = _run(kind, d, 2, rule, "eta32_f32")
    assert out_d.dtype == dt and g_d["deta"].dtype == torch.float32
    assert torch.equal(out_l, out_d)
    for k in g_l:
        if k != "deta":
            assert torch.equal(g_l[k], g_d[k]), k
    dlr_ref = (g_d["deta"].double().cpu() * _coef(rule, K)).sum(-2)
    err = max_abs(g_l["deta"], dlr_ref)
    _say(f"  dlr vs rows of dense deta: max-abs {err:.3e}")
    assert err <= 1e-5 * max(1.0, float(dlr_ref.abs().max()))


@pytest.mark.parametrize("kind", ["linear", "mlp"])
@pytest.mark.parametrize("rule", ["layer", "causal"])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_lr_against_oracle(kind, rule, dt):
    """Outputs and every gradient, dlr included, against autograd of the
    oracle with lr as the leaf (eta = make_eta(lr))."""
    _say(f"{kind} lr {rule} {dt} vs oracle")
    FF = 256 if kind == "mlp" else 0
    B, H, NC = (1, 2, 5) if dt == torch.float32 else (2, 2, 12)
    d = _inputs(B, H, NC, 64, FF, dt, rule, seed=73)
    out, grads = _run(kind, d, 4, rule, "lr")
    ref = _oracle(kind, d, 0, rule)
    ref32 = _oracle(kind, d, 0, rule, torch.float32) if dt == torch.float32 else None
    grads["dlr"] = grads.pop("deta")
    bad = []
    for k, mine in [("out", out)] + sorted(grads.items()):
        r = ref[k]
        if dt == torch.float32:
            err, bound = max_abs(mine, r), fp32_bound(r, ref32[k])
        else:
            err, bound = rel_l2(mine, r), BF16_RTOL
        _say(f"  {k}: err {err:.3e} bound {bound:.3e}")
        if err > bound:
            bad.append(k)
    assert not bad
