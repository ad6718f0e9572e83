"""The producer/consumer kernels and the end-to-end forecaster on the HIP path
against the CPU oracle (oracle/ttt_layer_oracle.py, fp64).

Tolerances: fp32 activations max-abs 1e-4 for the elementwise kernels (they
compute in fp32; the observed error is ~1e-6); bf16 and fp16 activations rel-L2 2e-2 (the required bar); the
whole forecaster in fp32 rel-L2 per tensor within max(1e-4, C_FP32 times the
fp32 oracle's own rel-L2 error against fp64) (a composition of four kernels,
three GEMMs and the inner loop, each within fp32 rounding), in bf16 and fp16
rel-L2 2e-2 per tensor with the norm floor described at the test."""

import sys

import pytest
import torch

from oracle import ttt_layer_oracle as LO
from tests._util import C_FP32, max_abs, rel_l2

pytestmark = pytest.mark.gpu

FP32_ATOL = 1e-4
BF16_RTOL = 2e-2
FP32_RTOL_E2E = 1e-4
# bf16 bar for the tiny parameter gradients (norm below TINY times the
# largest parameter gradient's): the XU projection's (1e-4 of the largest at
# K = 64) enters only through the memory-cache gates, whose logit gradients
# are differences between readouts of nearly equal memo states, each formed
# with bf16 operands as the reference's readout forms them
# (kernels/mlp_cached_readout.py:97-101); the lr gate bias's (3e-3) is a sum
# over every token with cancellation.  Measured at K = 64: 0.15 and 0.02.
TINY = 1e-2
BF16_RTOL_TINY = 0.25


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _bound_ok(mine, ref, dt):
    if dt == torch.float32:
        err, bound = max_abs(mine, ref), FP32_ATOL
    else:
        err, bound = rel_l2(mine, ref), BF16_RTOL
    return err, bound


def _producer_case(B, L, H, F_, seed):
    g = torch.Generator().manual_seed(seed)
    D = H * F_
    ld = 4 * D + H + (-(4 * D + H)) % 8
    proj = torch.randn(B, L, ld, generator=g)
    proj[..., 4 * D + H:] = 0
    ln_w = 1 + 0.2 * torch.randn(H, F_, generator=g)
    ln_b = 0.2 * torch.randn(H, F_, generator=g)
    grads = [torch.randn(B, H, L // 16, 16, F_, generator=g) for _ in range(4)]
    dlr = torch.randn(B, H, L // 16, 16, generator=g)
    return proj, ln_w, ln_b, grads, dlr


def _oracle_producer(proj, ln_w, ln_b, H, F_, base_lr, grads, dlr):
    B, L, _ = proj.shape
    D = H * F_
    pj = proj.double().requires_grad_(True)
    lw, lb = ln_w.double().requires_grad_(True), ln_b.double().requires_grad_(True)
    parts = [pj[..., i * D:(i + 1) * D].reshape(B, L, H, F_) for i in range(4)]
    fr = LO.rope_freqs(F_, 1, 1, L)
    outs = LO.producer(*parts, pj[..., 4 * D:4 * D + H], fr, lw, lb, 16, base_lr)
    loss = sum((o * gr.double()).sum() for o, gr in zip(outs, list(grads) + [dlr]))
    loss.backward()
    return [o.detach() for o in outs], pj.grad, lw.grad, lb.grad


# model widths H*F of 256 and less, 384 and 1024: the backward's per-lane
# arrays come in one, two and four chunks of 256 features
@pytest.mark.parametrize("F_,H", [(64, 4), (32, 8), (64, 3), (64, 6), (64, 16)])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_producer_vs_oracle(F_, H, dt):
    from ttt_amd.layer_io import ProducerFunction, rope_table
    B, L, base_lr = 2, 64, 0.05
    _say(f"producer F{F_} H{H} {dt}")
    proj, ln_w, ln_b, grads, dlr = _producer_case(B, L, H, F_, seed=81)
    proj = proj.to(dt)
    ref, dproj_ref, dlw_ref, dlb_ref = _oracle_producer(proj, ln_w, ln_b, H, F_, base_lr,
                                                        [gr.to(dt) for gr in grads], dlr)
    dev = torch.device("cuda")
    pj = proj.to(dev).requires_grad_(True)
    lw, lb = ln_w.to(dev).requires_grad_(True), ln_b.to(dev).requires_grad_(True)
    outs = ProducerFunction.apply(pj, rope_table(F_, L).to(dev), lw, lb, H, 16, base_lr)
    loss = sum((o.float() * gr.to(dev).float()).sum() for o, gr in zip(outs, [gr.to(dt) for gr in grads] + [dlr]))
    loss.backward()
    torch.cuda.synchronize()
    bad = []
    for name, mine, r in zip(("XQ", "XK", "XV", "XU", "lr"), outs, ref):
        err, bound = _bound_ok(mine, r, dt if name != "lr" else torch.float32)
        _say(f"  {name}: err {err:.3e} bound {bound:.3e}")
        if err > bound:
            bad.append(name)
    D = H * F_
    for name, mine, r in (("dproj", pj.grad[..., :4 * D + H], dproj_ref[..., :4 * D + H]),
                          ("dln_w", lw.grad, dlw_ref), ("dln_b", lb.grad, dlb_ref)):
        err, bound = _bound_ok(mine, r, dt)
        _say(f"  {name}: err {err:.3e} bound {bound:.3e}")
        if err > bound:
            bad.append(name)
    assert not bad
    assert bool((pj.grad[..., 4 * D + H:] == 0).all())  # padding columns get a zero gradient


@pytest.mark.parametrize("F_,H", [(64, 4), (32, 8), (64, 8), (64, 12)])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_post_norm_vs_oracle(F_, H, dt):
    from ttt_amd.layer_io import PostNormFunction
    B, L = 2, 48
    D = H * F_
    _say(f"post-norm F{F_} H{H} {dt}")
    g = torch.Generator().manual_seed(83)
    x = torch.randn(B, H, L // 16, 16, F_, generator=g).to(dt)
    gamma, beta = 1 + 0.2 * torch.randn(D, generator=g), 0.2 * torch.randn(D, generator=g)
    dout = torch.randn(B, L, D, generator=g).to(dt)
    xr, gr, br = (t.double().requires_grad_(True) for t in (x, gamma, beta))
    ref = torch.nn.functional.layer_norm(xr.permute(0, 2, 3, 1, 4).reshape(B, L, D), (D,), gr, br, 1e-6)
    ref.backward(dout.double())
    dev = torch.device("cuda")
    xg, gg, bg = (t.to(dev).requires_grad_(True) for t in (x, gamma, beta))
    out = PostNormFunction.apply(xg, gg, bg)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    bad = []
    for name, mine, r in (("out", out, ref), ("dX", xg.grad, xr.grad), ("dgamma", gg.grad, gr.grad),
                          ("dbeta", bg.grad, br.grad)):
        err, bound = _bound_ok(mine, r.detach(), dt)
        _say(f"  {name}: err {err:.3e} bound {bound:.3e}")
        if err > bound:
            bad.append(name)
    assert not bad


def _forecaster(kind, B, L, H, F_, M, seed, K=16):
    from ttt_amd import series
    from ttt_amd.model import ModelConfig, TTTForecaster
    cfg = ModelConfig(seq_len=L, model_dim=H * F_, num_heads=H, ssm_layer=kind, mini_batch_size=K,
                      ttt_base_lr=0.05, mem_cache_segment_n_mini_batches=M, scan_checkpoint_group_size=16)
    torch.manual_seed(seed)
    model = TTTForecaster(cfg, d_in=7, d_out=7, pred_len=96)
    data = series.synthetic_series(seed=seed)
    x, y = series.batch(data, B, L, 96, 96, seed=seed)
    return cfg, model, x, y[:, -96:, :]


@pytest.mark.parametrize("kind,M,dt,K,F_", [("ttt_mlp", 2, torch.float32, 16, 64),
                                             ("ttt_mlp", 2, torch.bfloat16, 16, 64),
                                             ("ttt_linear", 0, torch.float32, 16, 64),
                                             ("ttt_mlp", 2, torch.float32, 64, 32),
                                             ("ttt_mlp", 2, torch.bfloat16, 64, 32),
                                             ("ttt_linear", 0, torch.float32, 64, 32),
                                             ("ttt_mlp", 2, torch.float16, 16, 64),
                                             ("ttt_mlp", 2, torch.float16, 64, 32),
                                             ("ttt_linear", 0, torch.float16, 64, 32)])
def test_forecaster_train_step_vs_oracle(kind, M, dt, K, F_):
    """One training step of the end-to-end forecaster at batch 2: the loss and
    the gradient of every parameter against the oracle in fp64 on the same
    weights and windows.  K = 16, F = 64 is the benchmark's shape (lookback
    512, horizon 96, 7 channels, H = 4 heads, memo segments of M = 2,
    checkpoint groups of 16); K = 64, F = 32 (model dim 128) is the
    reference's own ModelConfig / main.py shape, on the general-shape
    kernels.  fp16 runs as mixed-precision training does: fp16 autocast and a
    GradScaler (the loss scaled by 2^10, the gradients unscaled through
    the scaler, which must find no overflow)."""
    B, L, H = 2, 512, 4
    _say(f"forecaster {kind} M{M} {dt} B{B} L{L} H{H} F{F_} K{K}")
    cfg, model, x, y = _forecaster(kind, B, L, H, F_, M, seed=91, K=K)
    sd = {k: v.detach().double().requires_grad_(True) for k, v in model.state_dict().items()}
    pred = LO.forecaster_forward(sd, x.double(), cfg, 96, 7)
    loss_ref = torch.nn.functional.mse_loss(pred, y.double())
    loss_ref.backward()
    # fp32: the same oracle in fp32 measures what fp32 rounding alone does to
    # each gradient (the XU projection's, formed by cancellation through the
    # memory-cache gates, is the most sensitive)
    rtol32 = {}
    if dt == torch.float32:
        sd32 = {k: v.detach().float().requires_grad_(True) for k, v in model.state_dict().items()}
        torch.nn.functional.mse_loss(LO.forecaster_forward(sd32, x.float(), cfg, 96, 7), y.float()).backward()
        rtol32 = {k: rel_l2(sd32[k].grad, sd[k].grad) for k in sd if sd[k].grad is not None}
    dev = torch.device("cuda")
    model = model.to(dev)
    with torch.autocast("cuda", dtype=dt, enabled=dt != torch.float32):
        out = model(x.to(dev))
    loss = torch.nn.functional.mse_loss(out.float(), y.to(dev))
    if dt == torch.float16:
        opt = torch.optim.SGD(model.parameters(), lr=0.0)
        scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 10)
        scaler.scale(loss).backward()
        scaler.unscale_(opt)
        found = sum(float(v) for v in scaler._found_inf_per_device(opt).values())
        assert found == 0.0, "the scaled fp16 backward overflowed"
    else:
        loss.backward()
    torch.cuda.synchronize()
    tol = FP32_RTOL_E2E if dt == torch.float32 else BF16_RTOL
    err = abs(loss.item() - loss_ref.item()) / abs(loss_ref.item())
    _say(f"  loss {loss.item():.6f} vs {loss_ref.item():.6f}: rel {err:.3e}")
    bad = ["loss"] if err > tol else []
    # every parameter gradient by rel-L2 against its own norm; in bf16 and
    # fp16 the tiny ones (TINY) have the looser bar BF16_RTOL_TINY
    gmax = max(float(sd[n].grad.norm()) for n, _ in model.named_parameters() if sd[n].grad is not None)
    for name, prm in model.named_parameters():
        r = sd[name].grad
        if r is None:
            assert prm.grad is None or float(prm.grad.abs().max()) == 0.0, name
            continue
        e = rel_l2(prm.grad, r)
        if dt == torch.float32:
            tp = max(tol, C_FP32 * rtol32[name])
        else:
            tp = BF16_RTOL_TINY if float(r.norm()) < TINY * gmax else tol
        _say(f"  d{name}: rel-L2 {rel_l2(prm.grad, r):.3e} (|ref| {float(r.norm()):.3e}), bound ratio {e / tp:.2f}")
        if e > tp:
            bad.append(name)
    assert not bad


def test_forecaster_step_in_a_graph_matches_eager():
    """The config-4 training step (forward, loss, backward, gradient clipping,
    AdamW) and an inference forward captured once each in a HIP graph
    (torch.cuda.CUDAGraph): every replay, with eager steps of a copy of the
    model between the replays, matches those eager steps (loss, every
    parameter, the inference output).  The library's launches go to the
    current stream and allocate nothing outside torch, so they capture."""
    import copy
    B, L, H, F_ = 2, 512, 4, 64
    _say(f"forecaster graph B{B} L{L} H{H} F{F_}")
    cfg, model, x, y = _forecaster("ttt_mlp", B, L, H, F_, 2, seed=93)
    dev = torch.device("cuda")
    model = model.to(dev)
    sx, sy = x.to(dev), y.to(dev)
    model_e = copy.deepcopy(model)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=1e-2, capturable=True)
    opt_e = torch.optim.AdamW(model_e.parameters(), lr=1e-3, weight_decay=1e-2, capturable=True)

    def step(m, o):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            pred = m(sx)
        loss = torch.nn.functional.mse_loss(pred.float(), sy)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(m.parameters(), 1.0)
        o.step()
        return loss

    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            opt.zero_grad(set_to_none=True)
            step(model, opt)
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(2):
        opt_e.zero_grad(set_to_none=True)
        step(model_e, opt_e)
    g = torch.cuda.CUDAGraph()
    opt.zero_grad(set_to_none=True)
    with torch.cuda.graph(g):
        sloss = step(model, opt)
    for r in range(3):
        g.replay()
        opt_e.zero_grad(set_to_none=True)
        le = step(model_e, opt_e)
        torch.cuda.synchronize()
        dl = abs(float(sloss.detach()) - float(le.detach())) / abs(float(le.detach()))
        with torch.no_grad():
            dp = max(float((a - b).abs().max() / (b.abs().max() + 1e-12))
                     for a, b in zip(model.parameters(), model_e.parameters()))
        _say(f"  replay {r}: loss rel {dl:.2e}, parameters max rel {dp:.2e}")
        assert dl <= 1e-6 and dp <= 1e-6
    gi = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            model(sx)
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(gi):
            sout = model(sx)
        for r in range(2):
            gi.replay()
            eo = model_e(sx)  # the eager copy holds the same parameters
            torch.cuda.synchronize()
            d = float((sout.float() - eo.float()).abs().max() / (eo.float().abs().max() + 1e-12))
            _say(f"  inference replay {r}: max rel {d:.2e}")
            assert d <= 1e-6


@pytest.mark.parametrize("kind", ["ttt_mlp", "ttt_linear"])
def test_last_token_path_matches_full_output(kind):
    """TTTWrapper(last_only=True), the path the forecaster takes for its
    head, against the full [B, L, D] output's last row in fp32: the output and
    the gradient of every parameter under a loss on that row agree to fp32
    GEMM rounding (post-norm and `wo` run on the last mini-batch only; the
    other rows' outputs are never read, so their gradients are exact zeros)."""
    from ttt_amd.model import ModelConfig, TTTWrapper
    B, L, H, F_ = 2, 256, 4, 64
    _say(f"last-token path {kind} B{B} L{L} H{H} F{F_}")
    cfg = ModelConfig(seq_len=L, model_dim=H * F_, num_heads=H, ssm_layer=kind, mini_batch_size=16,
                      ttt_base_lr=0.05, mem_cache_segment_n_mini_batches=2 if kind == "ttt_mlp" else 0,
                      scan_checkpoint_group_size=16)
    torch.manual_seed(5)
    dev = torch.device("cuda")
    layer = TTTWrapper(cfg).to(dev)
    x = torch.randn(B, L, H * F_, device=dev)
    w = torch.randn(B, H * F_, device=dev)
    grads = []
    outs = []
    for last in (False, True):
        layer.zero_grad(set_to_none=True)
        h = layer(x, last_only=True) if last else layer(x)[:, -1]
        (h * w).sum().backward()
        outs.append(h.detach())
        grads.append({n: p.grad.detach().clone() for n, p in layer.named_parameters() if p.grad is not None})
    torch.cuda.synchronize()
    e = rel_l2(outs[1], outs[0])
    _say(f"  output rel-L2 {e:.2e}")
    assert e <= 1e-5
    assert grads[0].keys() == grads[1].keys()
    for n in grads[0]:
        e = rel_l2(grads[1][n], grads[0][n])
        _say(f"  d{n}: rel-L2 {e:.2e}")
        assert e <= 1e-5, n


@pytest.mark.parametrize("kind", ["ttt_mlp", "ttt_linear"])
def test_inference_forward_matches_training_forward(kind):
    """Under no_grad the inner-loop Functions skip the checkpoints, final
    state and saved buffer their backward would read; the layer's output is
    bitwise the training forward's."""
    from ttt_amd.model import ModelConfig, TTTWrapper
    B, L, H, F_ = 2, 256, 4, 64
    _say(f"inference forward {kind} B{B} L{L} H{H} F{F_}")
    cfg = ModelConfig(seq_len=L, model_dim=H * F_, num_heads=H, ssm_layer=kind, mini_batch_size=16,
                      ttt_base_lr=0.05, mem_cache_segment_n_mini_batches=2 if kind == "ttt_mlp" else 0,
                      scan_checkpoint_group_size=16)
    torch.manual_seed(7)
    dev = torch.device("cuda")
    layer = TTTWrapper(cfg).to(dev)
    x = torch.randn(B, L, H * F_, device=dev)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        with torch.no_grad():
            y_inf = layer(x)
        y_train = layer(x)
    torch.cuda.synchronize()
    assert y_train.requires_grad and not y_inf.requires_grad
    assert torch.equal(y_inf, y_train.detach())
