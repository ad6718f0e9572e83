"""TTT-MLP memory-cache combiner (ttt_mlp_memo_combine / _bwd) vs the CPU oracle.

The oracle (`memo_combine`, ttt_layer.py:506-561 restated) runs in fp64 on the
same (rounded) inputs.  Tolerances: fp32 max-abs <= 1e-4, or C_FP32 = 8 times
the fp32 oracle's own error against fp64 where that is larger
(tests/_util.fp32_bound); bf16 inputs rel-L2 <= 2e-2.  Gradients are those
of the oracle's autograd wrt XK, XU and XQW (the inputs the reference's loop
differentiates; XK only through each segment's current summary)."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import fp32_bound, max_abs, rel_l2

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _inputs(B, H, NC, F_, FF, M, seed, dtype=torch.float32, xu_scale=0.3):
    gen = torch.Generator().manual_seed(seed)
    NS = O.ceil_div(NC, M)
    r = lambda *s, sc=1.0: torch.randn(*s, generator=gen) * sc
    act = {"XQ": r(B, H, NC, 16, F_), "XK": r(B, H, NC, 16, F_), "XU": r(B, H, NC, 16, F_, sc=xu_scale),
           "XQW": r(B, H, NC, 16, F_)}
    d = {k: v.to(dtype) for k, v in act.items()}
    d.update({"W1": r(B, H, NS, F_, FF, sc=0.2), "b1": r(B, H, NS, 1, FF, sc=0.1),
              "W2": r(B, H, NS, FF, F_, sc=0.2), "b2": r(B, H, NS, 1, F_, sc=0.1),
              "ln_w": 1 + r(H, F_, sc=0.2), "ln_b": r(H, F_, sc=0.2), "dOut": r(B, H, NC, 16, F_).to(dtype)})
    return d


KEYS = ("XQ", "XK", "XU", "XQW", "W1", "b1", "W2", "b2", "ln_w", "ln_b")


GRADS = ("XK", "XU", "XQW")


def _oracle(d, M, dtype=torch.float64):
    a = {k: d[k].to(dtype) for k in KEYS}
    for k in GRADS:
        a[k].requires_grad_(True)
    out = O.memo_combine(*(a[k] for k in KEYS), M, dtype=dtype)
    out.backward(d["dOut"].to(dtype))
    return (out.detach(),) + tuple(a[k].grad for k in GRADS)


def _gpu(d, M):
    from ttt_amd.memo import mlp_memo_combine
    g = {k: d[k].cuda() for k in KEYS}
    for k in GRADS:
        g[k].requires_grad_(True)
    out = mlp_memo_combine(*(g[k] for k in KEYS), M)
    out.backward(d["dOut"].cuda())
    torch.cuda.synchronize()
    return (out.detach(),) + tuple(g[k].grad for k in GRADS)


@pytest.mark.parametrize("B,H,NC,F_,FF,M", [
    (2, 2, 7, 64, 64, 2),     # ragged last segment, one chunk
    (1, 3, 37, 64, 256, 2),   # 3 chunks per chain, 19 memo states
    (2, 2, 19, 32, 128, 3),   # F = 32, ragged chunk and segment
    (1, 2, 9, 64, 256, 1),    # one mini-batch per segment
])
def test_memo_combine_fp32(B, H, NC, F_, FF, M):
    _say(f"memo combine fp32 B{B} H{H} NC{NC} F{F_} FF{FF} M{M}")
    d = _inputs(B, H, NC, F_, FF, M, seed=NC * 10 + M)
    out, dxk, dxu, dxqw = _gpu(d, M)
    ref, rdxk, rdxu, rdxqw = _oracle(d, M)
    r32 = _oracle(d, M, torch.float32)
    bad = []
    for name, a, b, b32 in (("out", out, ref, r32[0]), ("dXK", dxk, rdxk, r32[1]), ("dXU", dxu, rdxu, r32[2]),
                            ("dXQW", dxqw, rdxqw, r32[3])):
        err, bound = max_abs(a, b), fp32_bound(b, b32)
        _say(f"  {name}: max-abs {err:.3e} (bound {bound:.3e})")
        if err > bound:
            bad.append(name)
    assert not bad


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("FF", [64, 256])
def test_memo_combine_16bit(FF, dt):
    B, H, NC, F_, M = 2, 3, 40, 64, 2
    _say(f"memo combine {dt} NC{NC} FF{FF} M{M}")
    d = _inputs(B, H, NC, F_, FF, M, seed=7 + FF, dtype=dt)
    out, dxk, dxu, dxqw = _gpu(d, M)
    ref, rdxk, rdxu, rdxqw = _oracle(d, M)
    assert out.dtype == dt and dxu.dtype == dt and dxk.dtype == dt
    bad = []
    for name, a, b in (("out", out, ref), ("out - XQW", out.float().cpu() - d["XQW"].float(),
                                            ref - d["XQW"].double()),
                       ("dXK", dxk, rdxk), ("dXU", dxu, rdxu), ("dXQW", dxqw, rdxqw)):
        err = rel_l2(a, b)
        _say(f"  {name}: rel-L2 {err:.3e}")
        if err > BF16_RTOL:
            bad.append(name)
    assert not bad


def test_memo_combine_one_segment_is_identity():
    d = _inputs(1, 2, 5, 64, 64, 8, seed=3)
    out, dxk, dxu, dxqw = _gpu(d, 8)
    torch.testing.assert_close(out.cpu(), d["XQW"], rtol=0, atol=0)
    assert float(dxu.abs().max()) == 0.0
    assert float(dxk.abs().max()) == 0.0
    torch.testing.assert_close(dxqw.cpu(), d["dOut"], rtol=0, atol=0)


def test_memo_combine_deterministic():
    d = _inputs(1, 2, 21, 64, 256, 2, seed=4, dtype=torch.bfloat16)
    a = _gpu(d, 2)
    b = _gpu(d, 2)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_memo_combine_after_the_mlp_forward():
    """The drop-in flow of TTTMLP.ttt: TritonMLP.apply with memo segment size M,
    then the combiner over its output and memo, against the oracle chain."""
    from mlp_triton import TritonMLP
    from ttt_amd.memo import mlp_memo_combine
    B, H, NC, F_, FF, M, G = 1, 2, 10, 64, 256, 2, 4
    _say(f"TritonMLP + memo combine fp32 NC{NC} M{M}")
    d = O.make_inputs(B, H, NC, 16, F_, FF=FF, seed=12, dtype=torch.float32)
    gen = torch.Generator().manual_seed(13)
    XU = 0.3 * torch.randn(B, H, NC, 16, F_, generator=gen)
    g = {k: v.cuda() for k, v in d.items()}
    out, W1m, b1m, W2m, b2m = TritonMLP.apply(g["ln_w"], g["ln_b"], g["W1"], g["b1"], g["W2"], g["b2"],
                                              g["XQ"], g["XV"], g["XK"], g["eta"], G, M)
    comb = mlp_memo_combine(g["XQ"], g["XK"], XU.cuda(), out, W1m, b1m, W2m, b2m, g["ln_w"], g["ln_b"], M)
    torch.cuda.synchronize()
    full = O.mlp_forward_full(*(d[k].double() for k in ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK",
                                                          "eta")), G=G, M=M)
    ref = O.memo_combine(d["XQ"].double(), d["XK"].double(), XU.double(), full["out"], full["W1_memo"],
                         full["b1_memo"], full["W2_memo"], full["b2_memo"], d["ln_w"].double(), d["ln_b"].double(), M)
    f32 = O.mlp_forward_full(*(d[k].float() for k in ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK",
                                                        "eta")), G=G, M=M)
    ref32 = O.memo_combine(d["XQ"].float(), d["XK"].float(), XU.float(), f32["out"], f32["W1_memo"], f32["b1_memo"],
                           f32["W2_memo"], f32["b2_memo"], d["ln_w"].float(), d["ln_b"].float(), M,
                           dtype=torch.float32)
    err, bound = max_abs(comb, ref), fp32_bound(ref, ref32)
    _say(f"  max-abs {err:.3e} bound {bound:.3e}")
    assert err <= bound


@pytest.mark.parametrize("F_,FF,dt", [(64, 256, torch.bfloat16), (32, 64, torch.bfloat16),
                                     (64, 256, torch.float16)])
def test_memo_packed_images_match_the_converting_path(monkeypatch, F_, FF, dt):
    """16-bit activations: a workspace with room for the memo states' LDS images (written
    once by the forward, copied straight into LDS by both calls) gives bitwise
    the results of a gates-only workspace, where every workgroup converts each
    state it stages."""
    from ttt_amd import _lib
    from ttt_amd.memo import memo_combine_backward, memo_combine_forward
    lib = _lib.load()
    M = 3
    _say(f"memo packed vs converting F{F_} FF{FF} {dt}")
    d = _inputs(2, 3, 13, F_, FF, M, seed=F_ + FF, dtype=dt)
    g = {k: d[k].cuda() for k in KEYS}
    dout = d["dOut"].cuda()

    def run():
        out, gates = memo_combine_forward(*(g[k] for k in KEYS), M)
        grads = memo_combine_backward(g["XQ"], g["XU"], g["XQW"], g["W1"], g["b1"], g["W2"], g["b2"], g["ln_w"],
                                      g["ln_b"], M, gates, dout)
        torch.cuda.synchronize()
        return out, grads, gates.numel()

    out_p, gr_p, n_p = run()
    monkeypatch.setattr(lib, "ttt_mlp_memo_workspace_bytes",
                        lambda B, H, NC, K, F, FF, M, code: lib.ttt_mlp_memo_gates_bytes(B, H, NC, K, F, M))
    out_c, gr_c, n_c = run()
    assert n_p > n_c
    assert torch.equal(out_p, out_c)
    for a, b in zip(gr_p, gr_c):
        assert torch.equal(a, b)
