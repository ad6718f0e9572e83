"""ttt_mlp_bwd_noalloc (the backward with its workspace in the library's
static device scratch) against ttt_mlp_bwd with a caller-allocated
workspace, through the C ABI: every output bitwise equal, on two calls in a
row, the second on a smaller problem (so it runs on what the first left in
the scratch).  A problem larger than the scratch is refused on the host."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import to_dev

pytestmark = pytest.mark.gpu

KEYS = ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK", "eta")


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _outputs(B, H, NC, F_, FF, dt, dev):
    f32 = dict(device=dev, dtype=torch.float32)
    act = dict(device=dev, dtype=dt)
    return [torch.empty((B, H, NC, 16, F_), **act) for _ in range(3)] + [
        torch.empty((B, H, NC, 16, 16), **act), torch.empty((B, H, F_, FF), **f32), torch.empty((B, H, 1, FF), **f32),
        torch.empty((B, H, FF, F_), **f32), torch.empty((B, H, 1, F_), **f32), torch.empty((B, H, F_), **f32),
        torch.empty((B, H, F_), **f32)]


def _case(B, H, NC, F_, FF, G, dt, seed):
    """Run the forward, then both backwards on the same inputs; returns the
    two lists of outputs (dXQ, dXK, dXV, deta, dW1, db1, dW2, db2, dln_w, dln_b)."""
    from ttt_amd import _lib
    from ttt_amd._common import dtype_code, ptr, stream_of
    from ttt_amd.mlp import mlp_forward
    dev = torch.device("cuda")
    d = O.make_inputs(B, H, NC, 16, F_, FF=FF, seed=seed, dtype=dt, with_grad=True)
    g = to_dev(d)
    _, ck, _, last, saved = mlp_forward(*(g[k] for k in KEYS), G, want_ckpt=True, want_last=True, want_saved=True)
    lib = _lib.load()
    code = dtype_code(dt)
    common = [ptr(g["XQ"]), ptr(g["XK"]), ptr(g["XV"]), ptr(g["eta"]), ptr(g["ln_w"]), ptr(g["ln_b"]),
              *(ptr(t) if t is not None else None for t in ck), *(ptr(t) for t in last), ptr(g["dOut"]),
              B, H, NC, 16, F_, FF, G, code, _lib.ETA_DENSE, O.LN_EPS]
    ref = _outputs(B, H, NC, F_, FF, dt, dev)
    nws = lib.ttt_mlp_bwd_workspace_bytes(B, H, NC, 16, F_, FF, code)
    ws = torch.empty(nws, device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        st = lib.ttt_mlp_bwd(*common, *(ptr(t) for t in ref), ptr(saved), saved.numel(), ptr(ws), nws,
                             stream_of(dev))
    assert st == 0, st
    mine = _outputs(B, H, NC, F_, FF, dt, dev)
    with torch.cuda.device(dev):
        st = lib.ttt_mlp_bwd_noalloc(*common, *(ptr(t) for t in mine), ptr(saved), saved.numel(), stream_of(dev))
        assert st == 0, lib.ttt_error_string(st)
        # the fused workers' timeout word of that call, read from the static scratch
        st = lib.ttt_mlp_bwd_check(None, 0, B, H, NC, 16, F_, FF, code, stream_of(dev))
    assert st == 0, lib.ttt_error_string(st)
    torch.cuda.synchronize()
    return ref, mine


def test_noalloc_matches_the_workspace_entry_point():
    names = ("dXQ", "dXK", "dXV", "deta", "dW1", "db1", "dW2", "db2", "dln_w", "dln_b")
    # first call, then a smaller one (other shape and dtype) on the same scratch
    for B, H, NC, F_, FF, G, dt in ((2, 4, 32, 64, 256, 8, torch.bfloat16), (1, 3, 12, 32, 64, 4, torch.float32)):
        _say(f"noalloc vs workspace: B{B} H{H} NC{NC} F{F_} FF{FF} G{G} {dt}")
        ref, mine = _case(B, H, NC, F_, FF, G, dt, seed=B * 100 + NC)
        for n, a, b in zip(names, ref, mine):
            assert torch.equal(a, b), n


def test_noalloc_refuses_a_problem_larger_than_its_scratch():
    from ttt_amd import _lib
    lib = _lib.load()
    B, H, NC, F_, FF = 16, 12, 128, 64, 256  # 0.59 GB of workspace
    assert lib.ttt_mlp_bwd_workspace_bytes(B, H, NC, 16, F_, FF, 1) > _lib.MLP_BWD_NOALLOC_SCRATCH_BYTES
    P = 0x10000
    st = lib.ttt_mlp_bwd_noalloc(*([P] * 15), B, H, NC, 16, F_, FF, 8, 1, _lib.ETA_DENSE, 1e-8, *([P] * 10), P,
                                 1 << 40, None)
    assert st == _lib.STATUS_SCRATCH
    assert b"scratch" in lib.ttt_error_string(st)
