"""Parity at the benchmark's full size: B=16, H=12, T=2048 (NC=128 mini-batches
of K=16), F=64, bf16 activations with fp32 state; TTT-MLP with FF=256 and
checkpoint group 8, TTT-Linear with group 16.

The oracle needs about a second per chain at this length, so the full launch
(192 chains) is checked through properties that do not depend on its size, and against the
oracle on whole chains:
  * determinism: the same launch twice gives the same bits;
  * chain independence: the recurrence never mixes (batch, head) chains, so
    every per-chain output of the full launch (the readout, dXQ, dXV, dXK,
    deta and the gradient wrt the chain's initial state) equals, bit for bit,
    that chain's output in a launch of its batch row alone (H chains);
  * two whole chains (all 128 mini-batches, first and last of the grid)
    against the fp64 oracle at the bf16 bar, rel-L2 <= 2e-2, every output
    including the chain's LayerNorm-parameter gradient partials (the
    launchers' per-chain [B,H,F] values before the host's sum over B).
Both eta forms the reference builds are run: the causal expansion and the
layer's row-constant eta[i][j] = lr[j]/K (ttt_layer.py:306-309).  The memo combiner (memo segment M=8: 16 memo
states per chain) and the cached readout (one fixed state per chain) are
checked the same way at the same B, H, T."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import oracle_linear_grads, oracle_mlp_grads, rel_l2, to_dev

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2
B, H, NC, K, F = 16, 12, 128, 16, 64
ROWS = (0, B - 1)                 # batch rows launched on their own
CHAINS = ((0, 0), (B - 1, H - 1))  # (b, h) checked against the oracle


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _mlp(d, G):
    from ttt_amd.mlp import mlp_backward, mlp_forward
    g = to_dev(d)
    out, ck, _, last, saved = mlp_forward(*(g[k] for k in ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV",
                                                          "XK", "eta")),
                                          G, want_ckpt=True, want_last=True, want_saved=True, ckpt_w1_only=True)
    (dlw, dlb, dW1, db1, dW2, db2), (dxq, dxv, dxk, deta) = mlp_backward(
        g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck, last, saved, g["dOut"], G, sum_ln=False)
    torch.cuda.synchronize()
    return dict(out=out, dXQ=dxq, dXV=dxv, dXK=dxk, deta=deta, dW1=dW1, db1=db1, dW2=dW2, db2=db2,
                dln_w=dlw, dln_b=dlb)


def _linear(d, G):
    from ttt_amd.linear import linear_backward, linear_forward
    g = to_dev(d)
    out, (Wc, _), (Wl, _), saved = linear_forward(g["ln_w"], g["ln_b"], g["W1"], g["b1"], g["XQ"], g["XV"], g["XK"],
                                                  g["eta"], G, want_ckpt=True, want_last=True, want_saved=True)
    (dlw, dlb, dW, db), (dxq, dxv, dxk, deta) = linear_backward(
        g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], Wc, Wl, saved, g["dOut"], G, sum_ln=False)
    torch.cuda.synchronize()
    return dict(out=out, dXQ=dxq, dXV=dxv, dXK=dxk, deta=deta, dW1=dW, db1=db, dln_w=dlw, dln_b=dlb)


def _row(d, b):
    return {k: v if k in ("ln_w", "ln_b") else v[b:b + 1] for k, v in d.items()}


def _chain(d, b, h):
    return {k: v[h:h + 1] if k in ("ln_w", "ln_b") else v[b:b + 1, h:h + 1] for k, v in d.items()}


def _check(d, run, oracle, G):
    full = {k: v.cpu() for k, v in run(d, G).items()}
    again = {k: v.cpu() for k, v in run(d, G).items()}
    bad = [k for k in full if not torch.equal(full[k], again[k])]
    _say("  determinism: differing outputs", bad)
    assert not bad, f"not deterministic: {bad}"

    for b in ROWS:
        row = {k: v.cpu() for k, v in run(_row(d, b), G).items()}
        bad = []
        for k in row:
            same = torch.equal(row[k][0], full[k][b])
            if not same:
                diff = float((row[k][0].double() - full[k][b].double()).abs().max())
                bad.append(f"{k} (max diff {diff:.3e})")
        _say(f"  batch row {b} alone vs the full launch: differing", bad)
        assert not bad, f"chains of row {b} depend on the rest of the launch: {bad}"

    for b, h in CHAINS:
        dc = _chain(d, b, h)
        ref = oracle(dc, dc["dOut"], G=0)
        bad = []
        for k in full:
            err = rel_l2(full[k][b:b + 1, h:h + 1], ref[k])
            _say(f"  chain ({b},{h}) {k}: rel-L2 {err:.3e}")
            if err > BF16_RTOL:
                bad.append(k)
        assert not bad, f"chain ({b},{h}) off the oracle: {bad}"


@pytest.mark.parametrize("kind", ["causal", "layer"])
def test_mlp_fwd_bwd_full_size(kind):
    _say(f"mlp fwd+bwd full size B{B} H{H} NC{NC} F{F} FF256 G8 bf16, {kind} eta")
    d = O.make_inputs(B, H, NC, K, F, FF=256, seed=3, dtype=torch.bfloat16, with_grad=True, eta_kind=kind)
    _check(d, _mlp, oracle_mlp_grads, G=8)


@pytest.mark.parametrize("kind", ["causal", "layer"])
def test_linear_fwd_bwd_full_size(kind):
    _say(f"linear fwd+bwd full size B{B} H{H} NC{NC} F{F} G16 bf16, {kind} eta")
    d = O.make_inputs(B, H, NC, K, F, seed=2, dtype=torch.bfloat16, with_grad=True, eta_kind=kind)
    _check(d, _linear, oracle_linear_grads, G=16)


def _memo_inputs(seed):
    """XQ, XK, XU, XQW, dOut [B,H,NC,K,F] bf16 and 16 memo states per chain"""
    gen = torch.Generator().manual_seed(seed)
    NS, FF = NC // 8, 256
    r = lambda *s, sc=1.0: torch.randn(*s, generator=gen) * sc
    d = {"XQ": r(B, H, NC, K, F), "XK": r(B, H, NC, K, F), "XU": r(B, H, NC, K, F, sc=0.3),
         "XQW": r(B, H, NC, K, F), "dOut": r(B, H, NC, K, F)}
    d = {k: v.to(torch.bfloat16) for k, v in d.items()}
    d.update({"W1": r(B, H, NS, F, FF, sc=0.2), "b1": r(B, H, NS, 1, FF, sc=0.1),
              "W2": r(B, H, NS, FF, F, sc=0.2), "b2": r(B, H, NS, 1, F, sc=0.1),
              "ln_w": 1 + r(H, F, sc=0.2), "ln_b": r(H, F, sc=0.2)})
    return d


MEMO_KEYS = ("XQ", "XK", "XU", "XQW", "W1", "b1", "W2", "b2", "ln_w", "ln_b")
MEMO_GRADS = ("XK", "XU", "XQW")


def _memo(d, M):
    from ttt_amd.memo import mlp_memo_combine
    g = {k: d[k].cuda() for k in MEMO_KEYS}
    for k in MEMO_GRADS:
        g[k].requires_grad_(True)
    out = mlp_memo_combine(*(g[k] for k in MEMO_KEYS), M)
    out.backward(d["dOut"].cuda())
    torch.cuda.synchronize()
    res = {"out": out.detach().cpu()}
    res.update({"d" + k: g[k].grad.cpu() for k in MEMO_GRADS})
    return res


def _memo_oracle(d, M):
    a = {k: d[k].double() for k in MEMO_KEYS}
    for k in MEMO_GRADS:
        a[k].requires_grad_(True)
    out = O.memo_combine(*(a[k] for k in MEMO_KEYS), M)
    out.backward(d["dOut"].double())
    res = {"out": out.detach()}
    res.update({"d" + k: a[k].grad for k in MEMO_GRADS})
    return res


def test_memo_combine_full_size():
    M = 8
    _say(f"memo combine full size B{B} H{H} NC{NC} F{F} FF256 M{M} bf16")
    d = _memo_inputs(seed=21)
    full = _memo(d, M)
    again = _memo(d, M)
    bad = [k for k in full if not torch.equal(full[k], again[k])]
    _say("  determinism: differing outputs", bad)
    assert not bad
    for b in ROWS:
        row = _memo(_row(d, b), M)
        bad = [k for k in row if not torch.equal(row[k][0], full[k][b])]
        _say(f"  batch row {b} alone vs the full launch: differing", bad)
        assert not bad
    for b, h in CHAINS:
        ref = _memo_oracle(_chain(d, b, h), M)
        bad = []
        for k in full:
            mine, want = full[k][b:b + 1, h:h + 1], ref[k]
            if k == "out":  # the combination's own term, not hidden by XQW
                xqw = d["XQW"][b:b + 1, h:h + 1].double()
                mine, want = mine.double() - xqw, want - xqw
            err = rel_l2(mine, want)
            _say(f"  chain ({b},{h}) {k}: rel-L2 {err:.3e}")
            if err > BF16_RTOL:
                bad.append(k)
        assert not bad, f"chain ({b},{h}) off the oracle: {bad}"


def test_cached_readout_full_size():
    from ttt_amd.mlp import mlp_cached_readout
    _say(f"cached readout full size XQ [{B},{H},{NC},{K},{F}] FF256 bf16")
    gen = torch.Generator().manual_seed(22)
    args = [torch.randn(B, H, NC, K, F, generator=gen).to(torch.bfloat16),
            0.2 * torch.randn(B, H, F, 256, generator=gen), 0.1 * torch.randn(B, H, 1, 256, generator=gen),
            0.2 * torch.randn(B, H, 256, F, generator=gen), 0.1 * torch.randn(B, H, 1, F, generator=gen),
            1 + 0.2 * torch.randn(H, F, generator=gen), 0.2 * torch.randn(H, F, generator=gen)]
    run = lambda a: mlp_cached_readout(*(x.cuda() for x in a)).cpu()
    full = run(args)
    assert torch.equal(full, run(args))
    for b in ROWS:
        row = run([x[b:b + 1] if i < 5 else x for i, x in enumerate(args)])
        assert torch.equal(row[0], full[b]), f"row {b} alone differs"
    for b, h in CHAINS:
        one = [x[b:b + 1, h:h + 1] if i < 5 else x[h:h + 1] for i, x in enumerate(args)]
        ref = O.cached_readout(*(x.double() for x in one))
        xq = one[0].double()
        err = rel_l2(full[b:b + 1, h:h + 1].double() - xq, ref - xq)
        _say(f"  chain ({b},{h}) readout term: rel-L2 {err:.3e}")
        assert err <= BF16_RTOL
