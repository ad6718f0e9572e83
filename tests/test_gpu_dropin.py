"""The reference-shaped entry points (ops.ttt_linear, ops.ttt_mlp,
TritonLinear.apply, TritonMLP.apply) through torch autograd on the GPU, vs
autograd of the oracle.  fp32 max-abs <= 1e-4, or C_FP32 = 8 times the fp32
oracle's own error against fp64 where that is larger (tests/_util.fp32_bound);
bf16 rel-L2 <= 2e-2."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import eta_own_dtype, fp32_bound, max_abs, rel_l2

pytestmark = pytest.mark.gpu

LIN = ["XK", "XQ", "XV", "eta", "ln_w", "ln_b", "W1", "b1"]
MLP = LIN + ["W2", "b2"]


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _grads(fn, d, names, dout_perm, dev):
    args = {n: d[n].to(dev).requires_grad_(True) for n in names}
    out = fn(args)
    out.backward(dout_perm.to(dev))
    res = {"out": out.detach()}
    res.update({"d" + n: args[n].grad for n in names})
    return res


def _oracle(fn, d, names, dout_perm, dtype=torch.float64):
    args = {n: d[n].to(dtype).requires_grad_(True) for n in names}
    out = fn(args)
    out.backward(dout_perm.to(dtype))
    res = {"out": out.detach()}
    res.update({"d" + n: args[n].grad for n in names})
    return res


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("which", ["ops.ttt_linear", "TritonLinear", "ops.ttt_mlp", "TritonMLP"])
def test_dropin_autograd(which, dt):
    import ops
    from linear_triton import TritonLinear
    from mlp_triton import TritonMLP
    _say(f"drop-in {which} {dt}")
    mlp = "mlp" in which.lower()
    B, H, NC, G = 2, 2, 5, 2
    d = eta_own_dtype(O.make_inputs(B, H, NC, 16, 64, FF=128 if mlp else 0, seed=40, dtype=dt, with_grad=True), dt)
    names = MLP if mlp else LIN
    if which.startswith("ops"):
        dperm = d["dOut"].permute(0, 2, 3, 1, 4)
        f_gpu = (lambda a: ops.ttt_mlp(*[a[n] for n in names], G)) if mlp else \
            (lambda a: ops.ttt_linear(*[a[n] for n in names], G))
        f_ref = (lambda a: O.ttt_mlp(*[a[n] for n in names], G)) if mlp else \
            (lambda a: O.ttt_linear(*[a[n] for n in names], G))
    else:
        dperm = d["dOut"]
        order = ["ln_w", "ln_b", "W1", "b1"] + (["W2", "b2"] if mlp else []) + ["XQ", "XV", "XK", "eta"]
        if mlp:
            f_gpu = lambda a: TritonMLP.apply(*[a[n] for n in order], G, 0)[0]  # noqa: E731
        else:
            f_gpu = lambda a: TritonLinear.apply(*[a[n] for n in order], G)  # noqa: E731
        base = (lambda a: O.ttt_mlp(*[a[n] for n in names], G)) if mlp else \
            (lambda a: O.ttt_linear(*[a[n] for n in names], G))
        f_ref = lambda a: base(a).permute(0, 3, 1, 2, 4)  # noqa: E731
    mine = _grads(f_gpu, d, names, dperm, "cuda")
    ref = _oracle(f_ref, d, names, dperm)
    ref32 = _oracle(f_ref, d, names, dperm, torch.float32) if dt == torch.float32 else None
    # output and input gradients come back in each input's dtype
    for k in ref:
        src = "XQ" if k == "out" else k[1:]
        assert mine[k].dtype == d[src].dtype, (k, mine[k].dtype)
        assert mine[k].shape == ref[k].shape, (k, mine[k].shape, ref[k].shape)
    bad = []
    for k in ref:
        if dt == torch.float32:
            err, bound = max_abs(mine[k], ref[k]), fp32_bound(ref[k], ref32[k])
        else:
            err, bound = rel_l2(mine[k], ref[k]), 2e-2
        _say(f"  {k}: {err:.3e} (bound {bound:.3e})")
        if err > bound:
            bad.append(k)
    assert not bad


def test_tritonmlp_memo_outputs():
    """TritonMLP.apply returns fp32, non-differentiable memo snapshots
    [B,H,ceil(NC/M),...] equal to the oracle's states after mini-batch s*M."""
    from mlp_triton import TritonMLP
    B, H, NC, M, G = 1, 2, 7, 3, 2
    d = O.make_inputs(B, H, NC, 16, 64, FF=256, seed=41, dtype=torch.float32)
    g = {k: v.cuda() for k, v in d.items()}
    outs = TritonMLP.apply(g["ln_w"], g["ln_b"], g["W1"], g["b1"], g["W2"], g["b2"], g["XQ"], g["XV"],
                           g["XK"], g["eta"], G, M)
    assert len(outs) == 5
    keys = ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK", "eta")
    ref = O.mlp_forward_full(*(d[k].double() for k in keys), G=G, M=M)
    ref32 = O.mlp_forward_full(*(d[k].float() for k in keys), G=G, M=M)
    for t, n in zip(outs[1:], ("W1", "b1", "W2", "b2")):
        assert t.dtype == torch.float32 and not t.requires_grad
        assert t.shape[2] == -(-NC // M)
        assert max_abs(t, ref[n + "_memo"]) <= fp32_bound(ref[n + "_memo"], ref32[n + "_memo"])
    assert TritonMLP.sharded_mode is False
