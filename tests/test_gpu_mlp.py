"""TTT-MLP HIP kernels vs the CPU oracle (forward, side outputs, backward,
cached readout).  Tolerances as for TTT-Linear: fp32 max-abs <= 1e-4, or
C_FP32 = 8 times the fp32 oracle's own error against fp64 where that is
larger (tests/_util.fp32_bound); bf16 rel-L2 <= 2e-2."""

import sys

import pytest
import torch

from oracle import ttt_oracle as O
from tests._util import FP32_ATOL, eta_own_dtype, fp32_bound, max_abs, oracle_mlp_grads, rel_l2, to_dev

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


KEYS = ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK", "eta")


def _fwd(d, G, M=0, want_saved=True):
    """(out, ckpt, memo, last, saved) of the HIP forward"""
    from ttt_amd.mlp import mlp_forward
    g = to_dev(d)
    return mlp_forward(*(g[k] for k in KEYS), G, M=M, want_ckpt=True, want_last=True, want_saved=want_saved)


def _perturb(d, H, F_, FF, seed):
    gen = torch.Generator().manual_seed(seed)
    d["ln_w"] = 1 + 0.2 * torch.randn(H, F_, generator=gen)
    d["ln_b"] = 0.2 * torch.randn(H, F_, generator=gen)
    d["b1"] = 0.1 * torch.randn(*d["b1"].shape, generator=gen)
    d["b2"] = 0.1 * torch.randn(*d["b2"].shape, generator=gen)
    return d


@pytest.mark.parametrize("FF", [64, 128, 256])
def test_mlp_fwd_fp32(FF):
    _say("mlp fwd fp32 FF", FF)
    d = _perturb(O.make_inputs(2, 2, 6, 16, 64, FF=FF, seed=1, dtype=torch.float32), 2, 64, FF, 3)
    out, ck, memo, last, _ = _fwd(d, G=4, M=2)
    ref = O.mlp_forward_full(*(d[k].double() for k in KEYS), G=4, M=2)
    ref32 = O.mlp_forward_full(*(d[k].float() for k in KEYS), G=4, M=2)
    bad = []
    for name, mine in (("out", out), ("W1_last", last[0]), ("b1_last", last[1]), ("W2_last", last[2]),
                       ("b2_last", last[3]), ("W1_ckpt", ck[0]), ("b1_ckpt", ck[1]), ("W2_ckpt", ck[2]),
                       ("b2_ckpt", ck[3]), ("W1_memo", memo[0]), ("b1_memo", memo[1]), ("W2_memo", memo[2]),
                       ("b2_memo", memo[3])):
        err, bound = max_abs(mine, ref[name]), fp32_bound(ref[name], ref32[name])
        _say(f"  {name}: max-abs {err:.3e} bound {bound:.3e}")
        if err > bound:
            bad.append(name)
    assert not bad


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("kind", ["causal", "layer"])
def test_mlp_fwd_16bit_ff256(kind, dt):
    _say("mlp fwd FF256", dt, kind)
    d = O.make_inputs(2, 3, 24, 16, 64, FF=256, seed=2, dtype=dt, eta_kind=kind)
    out, ck, memo, last, _ = _fwd(d, G=8, M=2)
    ref = O.mlp_forward_full(*(d[k].double() for k in KEYS), G=8, M=2)
    bad = []
    for name, mine in (("out", out), ("W1_last", last[0]), ("W2_last", last[2]), ("W1_ckpt", ck[0]),
                       ("W2_memo", memo[2])):
        err = rel_l2(mine, ref[name])
        _say(f"  {name}: rel-L2 {err:.3e}")
        if err > BF16_RTOL:
            bad.append(name)
    assert not bad


def test_mlp_fwd_headdim32():
    _say("mlp fwd fp32 F32 FF64")
    d = O.make_inputs(1, 2, 5, 16, 32, FF=64, seed=4, dtype=torch.float32)
    out, _, _, last, _ = _fwd(d, G=2)
    ref = O.mlp_forward_full(*(d[k].double() for k in KEYS), G=2)
    assert max_abs(out, ref["out"]) <= FP32_ATOL
    assert max_abs(last[2], ref["W2_last"]) <= FP32_ATOL


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_mlp_fwd_saved_buffer(dt):
    """Saving for the backward leaves every forward output unchanged; the saved
    bias decrements add up to the bias change over the sequence,
    b_init - sum_s b_dec[s] = b_last; the saved update operand -e*G1 is -e
    times the saved G1."""
    _say("mlp fwd saved buffer", dt)
    B, H, NC, F_, FF = 2, 2, 7, 64, 128
    d = _perturb(O.make_inputs(B, H, NC, 16, F_, FF=FF, seed=11, dtype=dt), H, F_, FF, 12)
    out0, ck0, _, last0, none = _fwd(d, G=3, want_saved=False)
    out1, ck1, _, last1, saved = _fwd(d, G=3)
    assert none is None
    assert torch.equal(out0, out1)
    for a, b in zip(ck0 + last0, ck1 + last1):
        assert torch.equal(a, b)
    st = 4 if dt == torch.float32 else 2
    slot = (7 * FF + F_) * 16 * st + (FF + F_) * 4 + 3 * F_ * 64 + 4096
    assert saved.numel() == B * H * NC * slot
    u = saved.view(B * H, NC, slot)
    b1d = u[:, :, (FF + F_) * 16 * st:(FF + F_) * 16 * st + FF * 4].contiguous().view(torch.float32)
    b2d = u[:, :, (FF + F_) * 16 * st + FF * 4:(FF + F_) * 16 * st + (FF + F_) * 4].contiguous().view(torch.float32)
    g = to_dev(d)
    b1 = g["b1"].reshape(B * H, FF) - b1d.sum(1)
    b2 = g["b2"].reshape(B * H, F_) - b2d.sum(1)
    assert max_abs(b1, last1[1].reshape(B * H, FF)) <= 1e-5 * max(1.0, float(b1.abs().max()))
    assert max_abs(b2, last1[3].reshape(B * H, F_)) <= 1e-5 * max(1.0, float(b2.abs().max()))
    # the update operand -e*G1 and the saved G1 agree: both hidden-wide regions
    # hold, for wave w, tile o and lane l = 16 g + n, four values (j) of row
    # t = 4 g + j, hidden unit 64 w + 16 o + n
    def hidden(off):
        r = u[:, :, off:off + FF * 16 * st].contiguous().view(dt_).float()
        r = r.reshape(B * H, NC, FF // 64, 4, 4, 16, 4)      # [chain, s, w, o, g, n, j]
        return r.permute(0, 1, 4, 6, 2, 3, 5).reshape(B * H, NC, 16, FF)
    dt_ = dt
    g1e = hidden(0)
    g1 = hidden((FF + F_) * 16 * st + (FF + F_) * 4 + 2 * FF * 16 * st)
    e = g["eta"].reshape(B * H, NC, 16, 16)[:, :, 15, :].float()
    ref = -e[..., None] * g1
    tol = 1e-2 if st == 2 else 1e-6
    assert float((g1e - ref).abs().max()) <= tol * max(1.0, float(ref.abs().max()))


def _bwd(d, G):
    from ttt_amd.mlp import mlp_backward
    g = to_dev(d)
    out, ck, _, last, saved = _fwd(d, G)
    (dlw, dlb, dW1, db1, dW2, db2), (dxq, dxv, dxk, deta) = mlp_backward(
        g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck, last, saved, g["dOut"], G)
    return dict(dXQ=dxq, dXV=dxv, dXK=dxk, deta=deta, dW1=dW1, db1=db1, dW2=dW2, db2=db2, dln_w=dlw, dln_b=dlb)


@pytest.mark.parametrize("FF", [64, 256])
def test_mlp_bwd_fp32(FF):
    _say("mlp bwd fp32 FF", FF)
    d = _perturb(O.make_inputs(1, 2, 5, 16, 64, FF=FF, seed=5, dtype=torch.float32, with_grad=True), 2, 64, FF, 6)
    mine = _bwd(d, G=2)
    ref = oracle_mlp_grads(d, d["dOut"], G=0)
    ref32 = oracle_mlp_grads(d, d["dOut"], G=0, dtype=torch.float32)
    bad = []
    for k in mine:
        err, bound = max_abs(mine[k], ref[k]), fp32_bound(ref[k], ref32[k])
        _say(f"  {k}: max-abs {err:.3e} bound {bound:.3e} rel-L2 {rel_l2(mine[k], ref[k]):.3e}")
        if err > bound:
            bad.append(k)
    assert not bad


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_mlp_bwd_16bit_ff256(dt):
    _say("mlp bwd FF256", dt)
    d = eta_own_dtype(O.make_inputs(2, 2, 16, 16, 64, FF=256, seed=7, dtype=dt, with_grad=True), dt)
    mine = _bwd(d, G=8)
    ref = oracle_mlp_grads(d, d["dOut"], G=0)
    bad = []
    for k in mine:
        err = rel_l2(mine[k], ref[k])
        _say(f"  {k}: rel-L2 {err:.3e}")
        if err > BF16_RTOL:
            bad.append(k)
    assert not bad


@pytest.mark.parametrize("NC,G,F_,FF,dt", [
    (1, 1, 64, 256, torch.float32),
    (7, 3, 64, 128, torch.float32),
    (6, 4, 32, 64, torch.float32),
    (1, 1, 64, 256, torch.bfloat16),
    (9, 4, 32, 128, torch.bfloat16),
    (9, 4, 32, 128, torch.float16),
    (5, 2, 64, 64, torch.float16),
])
def test_mlp_bwd_edges(NC, G, F_, FF, dt):
    """single mini-batch, group sizes that do not divide NC, F = 32, FF = 64/128"""
    _say(f"mlp bwd NC{NC} G{G} F{F_} FF{FF} {dt}")
    d = _perturb(eta_own_dtype(O.make_inputs(1, 2, NC, 16, F_, FF=FF, seed=30 + NC, dtype=dt, with_grad=True), dt),
                 2, F_, FF, 31)
    mine = _bwd(d, G=G)
    ref = oracle_mlp_grads(d, d["dOut"], G=0)
    ref32 = oracle_mlp_grads(d, d["dOut"], G=0, dtype=torch.float32) if dt == torch.float32 else None
    bad = []
    for k in mine:
        if dt == torch.float32:
            err, bound = max_abs(mine[k], ref[k]), fp32_bound(ref[k], ref32[k])
        else:
            err, bound = rel_l2(mine[k], ref[k]), BF16_RTOL
        _say(f"  {k}: err {err:.3e} bound {bound:.3e}")
        if err > bound:
            bad.append(k)
    assert not bad


@pytest.mark.parametrize("F_,FF", [(64, 256), (32, 128)])
def test_mlp_bwd_fused_workers_finish_every_group(F_, FF):
    """Where the dXQ/dXK pass runs inside the sweep's launch (as many waves per
    chain as feature tiles), every (chain, checkpoint group) flag is raised,
    every task was taken and no worker gave up waiting; the gradients match a
    run whose workspace held stale control words from an earlier call."""
    from ttt_amd import _lib
    from ttt_amd.mlp import mlp_backward
    B, H, NC, G = 2, 3, 11, 4
    NK = -(-NC // G)
    _say(f"fused dXQ/dXK workers bf16 F{F_} FF{FF} NC{NC} G{G}")
    d = O.make_inputs(B, H, NC, 16, F_, FF=FF, seed=31, dtype=torch.bfloat16, with_grad=True)
    out, ck, _, last, saved = _fwd(d, G)
    g = to_dev(d)
    lib = _lib.load()
    nws = lib.ttt_mlp_bwd_workspace_bytes(B, H, NC, 16, F_, FF, 1)
    ws = torch.full((nws,), 0x7F, device="cuda", dtype=torch.uint8)  # stale control words
    args = (g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck, last, saved, g["dOut"], G)
    first = mlp_backward(*args, workspace=ws)
    torch.cuda.synchronize()
    slot = 2 * FF * 16 * 2 + 2 * F_ * 64
    ctrl = ws[B * H * NC * slot:].view(torch.int32).cpu()
    ntask = B * H * NK
    assert int(ctrl[1]) == 0, "a worker timed out waiting for a group"
    assert int(ctrl[0]) >= ntask
    assert bool((ctrl[4:4 + ntask] == 1).all())
    second = mlp_backward(*args, workspace=ws)
    torch.cuda.synchronize()
    for a, b in zip(first[0] + first[1], second[0] + second[1]):
        assert torch.equal(a, b)


def test_mlp_bwd_more_chains_than_cus():
    """More chains than the device has CUs to spare: the dXQ/dXK pass of the
    4-wave shape falls back to its own launch after the sweeps."""
    B, H, NC, G = 66, 4, 3, 2  # 264 chains
    _say(f"mlp bwd bf16 B{B} H{H} NC{NC} (two launches)")
    d = O.make_inputs(B, H, NC, 16, 64, FF=256, seed=51, dtype=torch.bfloat16, with_grad=True)
    mine = _bwd(d, G=G)
    ref = oracle_mlp_grads(d, d["dOut"], G=0)
    bad = []
    for k in mine:
        err = rel_l2(mine[k], ref[k])
        _say(f"  {k}: rel-L2 {err:.3e}")
        if err > BF16_RTOL:
            bad.append(k)
    assert not bad


def test_mlp_bwd_worker_timeout_is_loud():
    """With the poll limit set to 0 from the host, a fused dXQ/dXK worker
    whose checkpoint group is not yet published gives up at once (every
    kernel still exits normally): its group's dXQ and dXK rows hold NaN and
    ttt_mlp_bwd_check reports the timeout, so wrong gradients never pass
    silently.  Groups computed before giving up, and everything the reverse
    sweep writes itself, equal a normal run bit for bit.  With the fused mode
    switched off (two launches) the gradients equal the fused run's."""
    from ttt_amd import _lib
    from ttt_amd.mlp import mlp_backward, mlp_bwd_status
    B, H, NC, G, F_, FF = 2, 4, 64, 4, 64, 256
    NK = NC // G
    _say(f"fused worker timeout: bf16 B{B} H{H} NC{NC} G{G} poll limit 0")
    d = O.make_inputs(B, H, NC, 16, F_, FF=FF, seed=61, dtype=torch.bfloat16, with_grad=True)
    out, ck, _, last, saved = _fwd(d, G)
    g = to_dev(d)
    lib = _lib.load()
    nws = lib.ttt_mlp_bwd_workspace_bytes(B, H, NC, 16, F_, FF, 1)
    ws = torch.empty(nws, device="cuda", dtype=torch.uint8)
    args = (g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck, last, saved, g["dOut"], G)
    good = mlp_backward(*args, workspace=ws, check_timeout=False)
    assert mlp_bwd_status(ws, B, H, NC, 16, F_, FF, 1) == 0
    old = _lib.get_option(_lib.OPT_MLP_BWD_POLL_LIMIT)
    try:
        _lib.set_option(_lib.OPT_MLP_BWD_POLL_LIMIT, 0)
        bad = mlp_backward(*args, workspace=ws, check_timeout=False)
        st = mlp_bwd_status(ws, B, H, NC, 16, F_, FF, 1)
    finally:
        _lib.set_option(_lib.OPT_MLP_BWD_POLL_LIMIT, old)
    assert st == _lib.STATUS_TIMEOUT
    # sweep outputs: dW1..db2, dln (first tuple), dXV and deta
    for a, b in zip(good[0], bad[0]):
        assert torch.equal(a, b)
    assert torch.equal(good[1][1], bad[1][1]) and torch.equal(good[1][3], bad[1][3])
    n_nan = 0
    for gi, bi in ((good[1][0], bad[1][0]), (good[1][2], bad[1][2])):  # dXQ, dXK
        gb = gi.reshape(B * H, NK, G * 16 * F_)
        bb = bi.reshape(B * H, NK, G * 16 * F_)
        for c in range(B * H):
            for k in range(NK):
                if torch.isnan(bb[c, k]).all():
                    n_nan += 1
                else:
                    assert torch.equal(gb[c, k], bb[c, k]), (c, k)
    _say(f"  {n_nan} of {2 * B * H * NK} (tensor, chain, group) blocks poisoned")
    assert n_nan > 0
    # the normal limit again: no timeout, same gradients
    again = mlp_backward(*args, workspace=ws, check_timeout=True)
    for a, b in zip(good[0] + good[1], again[0] + again[1]):
        assert torch.equal(a, b)
    # two launches instead of the fused workers
    try:
        _lib.set_option(_lib.OPT_MLP_BWD_FUSED, 0)
        two = mlp_backward(*args, workspace=ws, check_timeout=True)
    finally:
        _lib.set_option(_lib.OPT_MLP_BWD_FUSED, 1)
    for a, b in zip(good[0] + good[1], two[0] + two[1]):
        assert torch.equal(a, b)
