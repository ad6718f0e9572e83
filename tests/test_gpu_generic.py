"""The general-shape inner loops (mini-batch K in {16, 32, 48, 64}, hidden width FF =
F = 32 as the reference's TTTMLP builds it, F from 32 to 256, FF up to 1024) against the CPU oracle:
forward with every side output (out, final state, checkpoints, memo
snapshots) and the backward's gradients of every input.  The reference's own
model configuration (ModelConfig defaults, main.py: K = 64, model dim 128 over
4 heads so F = 32, FF = F) is among the cases.

Tolerances as for the specialised kernels: fp32 max-abs <= 1e-4, or 8 times
the fp32 oracle's own error against fp64 where that is larger
(tests/_util.fp32_bound); bf16 and fp16 rel-L2 <= 2e-2."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import eta_own_dtype, fp32_bound, max_abs, oracle_linear_grads, oracle_mlp_grads, rel_l2, to_dev

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2
MLP_KEYS = ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK", "eta")
LIN_KEYS = ("ln_w", "ln_b", "W1", "b1", "XQ", "XV", "XK", "eta")


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _perturb(d, H, F_, seed, mlp=True):
    gen = torch.Generator().manual_seed(seed)
    d["ln_w"] = 1 + 0.2 * torch.randn(H, F_, generator=gen)
    d["ln_b"] = 0.2 * torch.randn(H, F_, generator=gen)
    d["b1"] = 0.1 * torch.randn(*d["b1"].shape, generator=gen)
    if mlp:
        d["b2"] = 0.1 * torch.randn(*d["b2"].shape, generator=gen)
    return d


def _check(mine: dict, ref: dict, ref32, dt):
    bad = []
    for k, v in mine.items():
        if dt == torch.float32:
            err, bound = max_abs(v, ref[k]), fp32_bound(ref[k], ref32[k])
        else:
            err, bound = rel_l2(v, ref[k]), BF16_RTOL
        _say(f"  {k}: err {err:.3e} bound {bound:.3e}")
        if err > bound:
            bad.append(k)
    assert not bad


# (B, H, NC, K, F, FF, G, M, dtype, eta kind)
MLP_CASES = [
    (2, 4, 6, 64, 32, 32, 4, 2, torch.float32, "layer"),    # the reference's ModelConfig / main.py shape
    (2, 4, 6, 64, 32, 32, 4, 2, torch.bfloat16, "layer"),
    (1, 2, 4, 64, 64, 256, 3, 2, torch.float32, "causal"),
    (1, 2, 4, 64, 64, 256, 3, 3, torch.bfloat16, "causal"),
    (2, 2, 5, 32, 64, 64, 2, 2, torch.bfloat16, "causal"),
    (1, 3, 7, 16, 32, 32, 3, 2, torch.float32, "causal"),   # FF = 32 at K = 16
    (1, 2, 3, 48, 48, 96, 2, 1, torch.float32, "layer"),
    # the register-resident one-wave kernels' other mini-batch sizes (F = FF = 32)
    (1, 2, 5, 48, 32, 32, 2, 2, torch.float32, "causal"),
    (2, 2, 4, 32, 32, 32, 3, 1, torch.bfloat16, "layer"),
    (1, 2, 3, 16, 32, 32, 1, 3, torch.bfloat16, "causal"),
    # wide shapes: 16 columns per lane in the row passes (F > 64) and products
    # whose output is split into blocks of at most 480 rows and columns
    (1, 2, 3, 16, 128, 128, 2, 1, torch.float32, "causal"),
    (1, 1, 3, 32, 256, 256, 2, 2, torch.bfloat16, "causal"),
    (1, 2, 3, 64, 64, 512, 2, 2, torch.float32, "layer"),
    (1, 1, 2, 16, 64, 1024, 1, 1, torch.bfloat16, "causal"),
    (1, 1, 2, 64, 256, 768, 1, 1, torch.float32, "causal"),
    # fp16 activations: the reference's shape, a staged shape, a wide shape
    (2, 4, 6, 64, 32, 32, 4, 2, torch.float16, "layer"),
    (1, 2, 4, 64, 64, 256, 3, 3, torch.float16, "causal"),
    (1, 1, 3, 32, 128, 256, 2, 1, torch.float16, "causal"),
]


@pytest.mark.parametrize("B,H,NC,K,F_,FF,G,M,dt,kind", MLP_CASES)
def test_generic_mlp_forward(B, H, NC, K, F_, FF, G, M, dt, kind):
    from ttt_amd.mlp import mlp_forward
    _say(f"generic mlp fwd B{B} H{H} NC{NC} K{K} F{F_} FF{FF} G{G} M{M} {dt} {kind}")
    d = _perturb(O.make_inputs(B, H, NC, K, F_, FF=FF, seed=K + F_ + FF, dtype=dt, eta_kind=kind), H, F_, 7)
    g = to_dev(d)
    out, ck, memo, last, _ = mlp_forward(*(g[k] for k in MLP_KEYS), G, M=M, want_ckpt=True, want_last=True)
    torch.cuda.synchronize()
    ref = O.mlp_forward_full(*(d[k].double() for k in MLP_KEYS), G=G, M=M)
    ref32 = O.mlp_forward_full(*(d[k].float() for k in MLP_KEYS), G=G, M=M) if dt == torch.float32 else None
    mine = {"out": out}
    for i, nm in enumerate(("W1", "b1", "W2", "b2")):
        mine[nm + "_last"] = last[i]
        mine[nm + "_ckpt"] = ck[i]
        mine[nm + "_memo"] = memo[i]
    _check(mine, ref, ref32, dt)


@pytest.mark.parametrize("B,H,NC,K,F_,FF,G,M,dt,kind", MLP_CASES)
def test_generic_mlp_backward(B, H, NC, K, F_, FF, G, M, dt, kind):
    from ttt_amd.mlp import mlp_backward, mlp_forward
    _say(f"generic mlp bwd B{B} H{H} NC{NC} K{K} F{F_} FF{FF} G{G} {dt} {kind}")
    d = _perturb(eta_own_dtype(O.make_inputs(B, H, NC, K, F_, FF=FF, seed=K + F_ + FF + 1, dtype=dt, eta_kind=kind,
                                             with_grad=True), dt), H, F_, 8)
    g = to_dev(d)
    out, ck, _, last, saved = mlp_forward(*(g[k] for k in MLP_KEYS), G, want_ckpt=True, want_last=True,
                                          want_saved=True)
    (dlw, dlb, dW1, db1, dW2, db2), (dxq, dxv, dxk, deta) = mlp_backward(
        g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck, last, saved, g["dOut"], G)
    torch.cuda.synchronize()
    mine = dict(dXQ=dxq, dXV=dxv, dXK=dxk, deta=deta, dW1=dW1, db1=db1, dW2=dW2, db2=db2, dln_w=dlw, dln_b=dlb)
    ref = oracle_mlp_grads(d, d["dOut"], G=0)
    ref32 = oracle_mlp_grads(d, d["dOut"], G=0, dtype=torch.float32) if dt == torch.float32 else None
    _check(mine, ref, ref32, dt)


LIN_CASES = [
    (2, 4, 6, 64, 32, 4, torch.float32, "layer"),    # ModelConfig's default layer (ttt_linear) shape
    (2, 4, 6, 64, 32, 4, torch.bfloat16, "layer"),
    (1, 3, 5, 32, 64, 2, torch.float32, "causal"),
    (1, 2, 4, 16, 48, 3, torch.float32, "causal"),
    (1, 2, 3, 64, 64, 1, torch.bfloat16, "causal"),
    (1, 2, 3, 32, 128, 2, torch.float32, "causal"),
    (1, 3, 4, 48, 32, 3, torch.float32, "causal"),
    (2, 2, 5, 32, 32, 2, torch.bfloat16, "layer"),
    (1, 1, 3, 16, 256, 1, torch.bfloat16, "layer"),
    (2, 4, 6, 64, 32, 4, torch.float16, "layer"),
    (1, 2, 3, 32, 128, 2, torch.float16, "causal"),
]


@pytest.mark.parametrize("B,H,NC,K,F_,G,dt,kind", LIN_CASES)
def test_generic_linear_forward_backward(B, H, NC, K, F_, G, dt, kind):
    from ttt_amd.linear import linear_backward, linear_forward
    _say(f"generic linear B{B} H{H} NC{NC} K{K} F{F_} G{G} {dt} {kind}")
    d = _perturb(eta_own_dtype(O.make_inputs(B, H, NC, K, F_, seed=K + F_ + 3, dtype=dt, eta_kind=kind,
                                             with_grad=True), dt), H, F_, 9, mlp=False)
    g = to_dev(d)
    out, ck, last, saved = linear_forward(*(g[k] for k in LIN_KEYS), G, want_ckpt=True, want_last=True,
                                          want_saved=True)
    (dlw, dlb, dW1, db1), (dxq, dxv, dxk, deta) = linear_backward(
        g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck[0], last[0], saved, g["dOut"], G)
    torch.cuda.synchronize()
    ref = O.linear_forward_full(*(d[k].double() for k in LIN_KEYS), G=G)
    ref32 = O.linear_forward_full(*(d[k].float() for k in LIN_KEYS), G=G) if dt == torch.float32 else None
    _check({"out": out, "W1_last": last[0], "b1_last": last[1], "W1_ckpt": ck[0], "b1_ckpt": ck[1]}, ref, ref32, dt)
    gref = oracle_linear_grads(d, d["dOut"], G=0)
    gref32 = oracle_linear_grads(d, d["dOut"], G=0, dtype=torch.float32) if dt == torch.float32 else None
    _check(dict(dXQ=dxq, dXV=dxv, dXK=dxk, deta=deta, dW1=dW1, db1=db1, dln_w=dlw, dln_b=dlb), gref, gref32, dt)


@pytest.mark.parametrize("kind", ["layer", "causal"])
def test_generic_lr_rules_match_dense(kind):
    """lr [B,H,NC,K] expanded on chip by the rule equals the dense eta the host
    builds from the same lr (bitwise in fp32: the same coefficients), and dlr
    is the rule's contraction of the dense deta."""
    from ttt_amd.mlp import mlp_backward, mlp_forward
    B, H, NC, K, F_, FF, G = 1, 2, 3, 64, 32, 32, 2
    _say(f"generic lr rule {kind} K{K}")
    d = _perturb(O.make_inputs(B, H, NC, K, F_, FF=FF, seed=77, with_grad=True), H, F_, 10)
    gen = torch.Generator().manual_seed(78)
    lr = torch.sigmoid(torch.randn(B, H, NC, K, generator=gen)) / F_
    d["eta"] = O.eta_from_lr(lr, kind)
    g = to_dev(d)
    res = {}
    for rule, eta in (("dense", g["eta"]), (kind, lr.cuda())):
        out, ck, _, last, saved = mlp_forward(*(g[k] for k in MLP_KEYS[:-1]), eta, G, want_ckpt=True,
                                              want_last=True, want_saved=True, eta_rule=rule)
        grads = mlp_backward(g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], eta, ck, last, saved, g["dOut"], G,
                             eta_rule=rule)
        res[rule] = (out, grads)
    torch.cuda.synchronize()
    assert torch.equal(res["dense"][0], res[kind][0])
    deta = res["dense"][1][1][3].double().cpu()
    i = torch.arange(K, dtype=torch.float64)
    coef = (torch.full((K, K), 1.0 / K, dtype=torch.float64) if kind == "layer"
            else torch.tril(torch.ones(K, K, dtype=torch.float64)) / (i + 1)[:, None])
    dlr_ref = (deta * coef).sum(-2)
    assert max_abs(res[kind][1][1][3], dlr_ref) <= 1e-4 * max(1.0, float(dlr_ref.abs().max()))


@pytest.mark.parametrize("K", [64, 32])
@pytest.mark.parametrize("dt,eta", [(torch.float32, "dense"), (torch.bfloat16, "dense"), (torch.float16, "dense"),
                                    (torch.bfloat16, "layer"), (torch.float32, "causal")])
def test_small_mlp_backward_one_launch_matches_two(K, dt, eta):
    """The register-resident MLP backward with a minimal workspace (256
    bytes: one launch, every phase in the sweep) against the two-launch form
    (the readout path of every mini-batch first, then the sweeps), for the
    dense eta in the activation dtype, in fp32 (fp16: DENSE_F32) and the lr
    rules: the same gradients up to summation order (fp32 2e-5 relative,
    16-bit within the 2e-2 bar)."""
    from ttt_amd.mlp import mlp_backward, mlp_forward
    B, H, NC, F_, G = 2, 3, 5, 32, 2
    _say(f"small mlp bwd one vs two launches K{K} {dt} {eta}")
    d = _perturb(eta_own_dtype(O.make_inputs(B, H, NC, K, F_, FF=F_, seed=K + 7, dtype=dt, eta_kind="causal",
                                             with_grad=True), dt), H, F_, 13)
    if eta != "dense":
        gen = torch.Generator().manual_seed(K + 8)
        d["eta"] = torch.sigmoid(torch.randn(B, H, NC, K, generator=gen)) / F_
    g = to_dev(d)
    out, ck, _, last, saved = mlp_forward(*(g[k] for k in MLP_KEYS), G, want_ckpt=True, want_last=True,
                                          want_saved=True, eta_rule=eta)
    args = (g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck, last, saved, g["dOut"], G)
    two = mlp_backward(*args, eta_rule=eta)
    one = mlp_backward(*args, eta_rule=eta, workspace=torch.empty(256, device="cuda", dtype=torch.uint8))
    torch.cuda.synchronize()
    bound = 2e-5 if dt == torch.float32 else BF16_RTOL
    worst = max(rel_l2(a, b) for a, b in zip(one[0] + one[1], two[0] + two[1]))
    _say(f"  worst rel-L2 {worst:.3e} (bound {bound:.0e})")
    assert worst <= bound


@pytest.mark.parametrize("mlp,dt", [(True, torch.float32), (True, torch.bfloat16), (False, torch.float32),
                                    (True, torch.float16), (False, torch.float16)])
def test_small_kernels_match_the_staged_kernels(mlp, dt):
    """At the reference's model shape (K = 64, F = FF = 32) the register-
    resident kernels and the staged general-shape kernels (TTT_OPT_SMALL_KERNELS
    = 0) compute the same forward and gradients: fp32 to 2e-5 relative, bf16
    and fp16 within the 16-bit bar (different operand roundings)."""
    from ttt_amd import _lib
    from ttt_amd.linear import linear_backward, linear_forward
    from ttt_amd.mlp import mlp_backward, mlp_forward
    B, H, NC, K, F_, G = 2, 4, 5, 64, 32, 2
    _say(f"small vs staged {'mlp' if mlp else 'linear'} {dt}")
    d = _perturb(eta_own_dtype(O.make_inputs(B, H, NC, K, F_, FF=F_, seed=123, dtype=dt, eta_kind="causal",
                                             with_grad=True), dt), H, F_, 11, mlp=mlp)
    g = to_dev(d)
    res = []
    try:
        for small in (1, 0):
            _lib.set_option(_lib.OPT_SMALL_KERNELS, small)
            if mlp:
                out, ck, _, last, saved = mlp_forward(*(g[k] for k in MLP_KEYS), G, want_ckpt=True, want_last=True,
                                                      want_saved=True)
                grads = mlp_backward(g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck, last, saved,
                                     g["dOut"], G)
                flat = [out, *last, *grads[0], *grads[1]]
            else:
                out, ck, last, saved = linear_forward(*(g[k] for k in LIN_KEYS), G, want_ckpt=True, want_last=True,
                                                      want_saved=True)
                grads = linear_backward(g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck[0], last[0],
                                        saved, g["dOut"], G)
                flat = [out, *last, *grads[0], *grads[1]]
            torch.cuda.synchronize()
            res.append([t.detach().clone() for t in flat])
    finally:
        _lib.set_option(_lib.OPT_SMALL_KERNELS, 1)
    bound = 2e-5 if dt == torch.float32 else BF16_RTOL
    worst = max(rel_l2(a, b) for a, b in zip(*res))
    _say(f"  worst rel-L2 {worst:.3e} (bound {bound:.0e})")
    assert worst <= bound
