"""Fixed-weight TTT-MLP readout (ttt_mlp_cached_readout) vs the CPU oracle.

Tolerances: fp32 max-abs <= 1e-4 (scaled by the tensor's magnitude above 1);
bf16 rel-L2 <= 2e-2, measured on the readout term out - XQ so that the
residual does not hide its error."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import fp32_bound, max_abs, rel_l2

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _inputs(B, H, NS, F_, FF, seed, dtype=torch.float32, wscale=0.2):
    gen = torch.Generator().manual_seed(seed)
    XQ = torch.randn(B, H, NS, 16, F_, generator=gen).to(dtype)
    W1 = wscale * torch.randn(B, H, F_, FF, generator=gen)
    b1 = 0.1 * torch.randn(B, H, 1, FF, generator=gen)
    W2 = wscale * torch.randn(B, H, FF, F_, generator=gen)
    b2 = 0.1 * torch.randn(B, H, 1, F_, generator=gen)
    lw = 1 + 0.2 * torch.randn(H, F_, generator=gen)
    lb = 0.2 * torch.randn(H, F_, generator=gen)
    return [XQ, W1, b1, W2, b2, lw, lb]


def _gpu(args):
    from ttt_amd.mlp import mlp_cached_readout
    return mlp_cached_readout(*(a.cuda() for a in args))


@pytest.mark.parametrize("B,H,NS,F_,FF", [
    (2, 4, 17, 64, 256),   # 8 chains x 2 chunks (XCD-grouped block order), ragged last chunk
    (2, 4, 16, 64, 64),    # exactly one full chunk per chain
    (1, 3, 3, 32, 128),    # 3 chains (plain block order), partial waves
    (1, 1, 1, 64, 256),    # a single mini-batch
])
def test_readout_fp32(B, H, NS, F_, FF):
    _say(f"readout fp32 B{B} H{H} NS{NS} F{F_} FF{FF}")
    args = _inputs(B, H, NS, F_, FF, seed=B * 100 + NS)
    out = _gpu(args)
    ref = O.cached_readout(*(a.double() for a in args))
    ref32 = O.cached_readout(*(a.float() for a in args))
    err, bound = max_abs(out, ref), fp32_bound(ref, ref32)
    _say(f"  max-abs {err:.3e} bound {bound:.3e}")
    assert out.dtype == torch.float32 and out.shape == args[0].shape
    assert err <= bound


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("FF", [64, 256])
def test_readout_16bit(FF, dt):
    _say(f"readout {dt} FF{FF}")
    args = _inputs(2, 4, 5, 64, FF, seed=7, dtype=dt)
    out = _gpu(args)
    ref = O.cached_readout(*(a.double() for a in args))
    x = args[0].double()
    err = rel_l2(out.double().cpu() - x, ref - x)
    _say(f"  readout-term rel-L2 {err:.3e}")
    assert out.dtype == torch.float32
    assert err <= BF16_RTOL


def test_readout_memo_slices_in_place():
    """Memo snapshots from the forward, passed as W*_memo[:, :, j] views, give
    the oracle's readout with the oracle's memo state, and the same bits as a
    contiguous copy of the slice."""
    from ttt_amd.mlp import mlp_cached_readout, mlp_forward
    _say("readout from memo slices")
    B, H, NC, F_, FF, M = 2, 2, 6, 64, 256, 2
    d = O.make_inputs(B, H, NC, 16, F_, FF=FF, seed=5, dtype=torch.float32)
    keys = ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK", "eta")
    g = {k: v.cuda() for k, v in d.items()}
    _, _, memo, _, _ = mlp_forward(*(g[k] for k in keys), 3, M=M, want_ckpt=False)
    ref_full = O.mlp_forward_full(*(d[k].double() for k in keys), G=3, M=M)
    NS = memo[0].shape[2]
    for j in range(NS):
        seg = g["XQ"][:, :, j * M:(j + 1) * M]
        views = [m[:, :, j] for m in memo]
        assert not views[0].is_contiguous()
        out = mlp_cached_readout(seg, *views, g["ln_w"], g["ln_b"])
        out_c = mlp_cached_readout(seg, *(v.contiguous() for v in views), g["ln_w"], g["ln_b"])
        ref = O.cached_readout(d["XQ"][:, :, j * M:(j + 1) * M].double(),
                               *(ref_full[n + "_memo"][:, :, j] for n in ("W1", "b1", "W2", "b2")),
                               d["ln_w"].double(), d["ln_b"].double())
        ref32 = O.cached_readout(d["XQ"][:, :, j * M:(j + 1) * M].float(),
                                 *(ref_full[n + "_memo"][:, :, j].float() for n in ("W1", "b1", "W2", "b2")),
                                 d["ln_w"].float(), d["ln_b"].float())
        err, bound = max_abs(out, ref), fp32_bound(ref, ref32)
        _say(f"  slice {j}: max-abs {err:.3e} bound {bound:.3e}")
        assert torch.equal(out, out_c)
        assert err <= bound


def test_readout_dropin():
    from kernels.mlp_cached_readout import mlp_cached_readout_triton
    args = [a.cuda() for a in _inputs(1, 2, 2, 64, 256, seed=3, dtype=torch.bfloat16)]
    out = mlp_cached_readout_triton(*args)
    assert out.dtype == torch.float32 and out.shape == args[0].shape
    from ttt_amd.mlp import mlp_cached_readout
    assert torch.equal(out, mlp_cached_readout(*args))
