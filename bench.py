"""Throughput of the TTT-MLP / TTT-Linear inner loop on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--eta lr|dense]

Headline workload: TTT-MLP forward+backward, B=16, H=12,
T=2048 (NC=128 mini-batches of K=16), F=64, hidden 256, bf16 activations,
fp32 fast-weight state, checkpoints every G=8 mini-batches; eta is the
causal expansion eta[i][j] = lr[j]/(i+1) (j <= i) of the per-token learning
rate lr [B,H,NC,K] = sigmoid(u)/F, passed as the materialised [B,H,NC,K,K]
bf16 tensor (--eta lr passes lr itself, expanded on chip; the line reports
the other form too).  One step = the forward kernel
(writing the checkpoints and the saved buffer) + the backward kernel, the
launches TritonMLP.apply makes, on synthetic seeded inputs resident in HBM.

Every kernel launch is bracketed by HIP events on the stream it runs on, so
the per-kernel averages behind `roofline` come from the timed steps.
`roofline.traffic` (HBM bytes per launch) and `roofline.mfma_busy` (the
MFMA-busy fraction of the launch) are read from the committed rocprofv3
counter summaries under profiles/ when they exist for the kernel.

Also measured, one line each in the JSON: TTT-Linear fwd+bwd at the same
shape (G=16), TTT-MLP forward at B=8 (with and without memo M=2), TTT-Linear
forward fp32 at B2 H4 T256, the end-to-end forecaster (one AdamW training
step and inference at batch 32, lookback 512, horizon 96, 7 channels, H=4
heads of F=64, K=16, memo M=2, bf16 autocast), the cached readout and the
memory-cache combiner.

The CPU baselines time the oracle (the eager-PyTorch restatement of the
reference's ops path, fp32, autograd for the backward) on this host's usable
cores, on a bounded sample of each config's batch.

Other modes (for counter collection):
    --only mlp_fwd|mlp_bwd|linear_fwd|linear_bwd|readout|memo_fwd|memo_bwd|forecaster|forecaster_ref
    --copy-calibration     copy 1 GiB device-to-device (a kernel of known traffic)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "ttt-triton_amd")]

METRIC = "TTT-MLP/Linear fwd+bwd tokens/s (B16,H12,T2048,F64) + % MFMA/HBM roofline"
HBM_PEAK = 8.0e12          # B/s
MFMA_PEAK_BF16 = 2.5e15    # dense FLOP/s
MFMA_PEAK_F32 = 157.3e12
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.md")
COUNTER_FILE = os.path.join(ROOT, "profiles", "mfma_counters.md")

B, H, T, K, F, FF = 16, 12, 2048, 16, 64, 256
NC = T // K
G_MLP, G_LIN = 8, 16
MEMO_M = 8  # memo segment size (mini-batches) of the combiner leg
# the end-to-end forecaster (lookback 512, horizon 96, 7 channels, batch 32)
FC_B, FC_L, FC_H, FC_F, FC_PRED, FC_CH, FC_M, FC_G = 32, 512, 4, 64, 96, 7, 2, 16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-seconds", type=float, default=5.0, help="CPU time budget per config")
    ap.add_argument("--cpu-compile", action="store_true",
                    help="also time the headline CPU baseline (c3) with the oracle's mini-batch step under "
                         "torch.compile, as the reference's ops path compiles its own (ops/ttt_mlp.py:9); "
                         "compiling adds one to two minutes")
    ap.add_argument("--eta", choices=["lr", "dense"], default="dense")
    ap.add_argument("--only", choices=["mlp_fwd", "mlp_bwd", "linear_fwd", "linear_bwd", "readout", "memo_fwd",
                                       "memo_bwd", "forecaster", "forecaster_ref"])
    ap.add_argument("--copy-calibration", action="store_true")
    return ap.parse_args()


# ---------------------------------------------------------------- algorithmic counts
def mlp_state_floats(F_=F, FF_=FF):
    return 2 * F_ * FF_ + FF_ + F_


def lin_state_floats(F_=F):
    return F_ * F_ + F_


def mlp_fwd_flops(Bn=B, T_=T, F_=F, FF_=FF):
    return (14 * F_ * FF_ + 6 * K * FF_ + 6 * K * F_) * Bn * H * T_


def lin_fwd_flops(Bn=B, H_=H, T_=T, F_=F):
    return (6 * F_ * F_ + 6 * K * F_) * Bn * H_ * T_


def eta_bytes_per_token(eta):
    """dense: one row of the [K,K] eta per token (bf16); lr: one fp32 per token"""
    return K * 2 if eta == "dense" else 4


def fwd_bytes(state, G, ckpt, eta, Bn=B, H_=H, T_=T, F_=F, sx=2):
    """inputs XQ, XK, XV, eta read + out written + state read/written + checkpoints
    written (`ckpt` floats each: what the backward reads of the state)"""
    return (Bn * H_ * T_ * (4 * F_ * sx + eta_bytes_per_token(eta)) + Bn * H_ * state * 4 * 2
            + Bn * H_ * math.ceil(T_ // K / G) * ckpt * 4)


def bwd_bytes(state, G, ckpt, eta, Bn=B, H_=H, T_=T, F_=F, sx=2):
    """XQ, XK, XV, dout, eta read + dXQ, dXK, dXV, deta written + checkpoints read
    + state gradients written (and the per-chain LN partials)"""
    e = eta_bytes_per_token(eta)
    return (Bn * H_ * T_ * (4 * F_ * sx + e) + Bn * H_ * T_ * (3 * F_ * sx + e)
            + Bn * H_ * math.ceil(T_ // K / G) * ckpt * 4 + Bn * H_ * (state + 2 * F_) * 4 * 2)


def readout_flops():
    return 4 * F * FF * B * H * T


def readout_bytes(sx=2):
    return B * H * T * F * (sx + 4) + B * H * mlp_state_floats() * 4


# ---------------------------------------------------------------- inputs (seeded, on the CPU, then moved)
def make_inputs(torch, Bn, H_, NC_, F_, FF_=0, seed=0, dtype=None, eta="lr"):
    """XQ, XK, XV ~ N(0,1) [B,H,NC,K,F]; u ~ N(0,1) [B,H,NC,K] with
    lr = sigmoid(u)/F; W1 ~ N(0,0.02) [H,F,F or FF] (and W2 [H,FF,F]) tiled
    over B; biases 0, LN weight 1 / bias 0; dOut ~ N(0,1).  eta is lr
    (causal rule on chip) or the dense causal [B,H,NC,K,K] expansion."""
    dtype = dtype or torch.bfloat16
    gen = torch.Generator().manual_seed(seed)
    shp = (Bn, H_, NC_, K, F_)
    d = {n: torch.randn(shp, generator=gen).to(dtype) for n in ("XQ", "XK", "XV")}
    lr = torch.sigmoid(torch.randn((Bn, H_, NC_, K), generator=gen)) / F_
    hid = FF_ or F_
    d["W1"] = (0.02 * torch.randn((H_, F_, hid), generator=gen))[None].repeat(Bn, 1, 1, 1).contiguous()
    d["b1"] = torch.zeros(Bn, H_, 1, hid)
    if FF_:
        d["W2"] = (0.02 * torch.randn((H_, FF_, F_), generator=gen))[None].repeat(Bn, 1, 1, 1).contiguous()
        d["b2"] = torch.zeros(Bn, H_, 1, F_)
    d["dOut"] = torch.randn(shp, generator=gen).to(dtype)
    d["ln_w"], d["ln_b"] = torch.ones(H_, F_), torch.zeros(H_, F_)
    if eta == "lr":
        d["eta"] = lr
    else:
        i = torch.arange(K, dtype=torch.float32)
        scale = torch.tril(torch.ones(K, K)) / (i + 1)[:, None]
        d["eta"] = (lr[..., None, :] * scale).to(dtype)
    return d


class Timer:
    """HIP events on the launch stream around each named launch."""

    def __init__(self, torch):
        self.torch = torch
        self.marks = []

    def mark(self, name):
        ev = self.torch.cuda.Event(enable_timing=True)
        ev.record(self.torch.cuda.current_stream())
        self.marks.append((name, ev))

    def spans(self):
        self.torch.cuda.synchronize()
        out = {}
        for (name, a), (_, b) in zip(self.marks, self.marks[1:]):
            if name is not None:
                out.setdefault(name, []).append(a.elapsed_time(b) * 1e-3)
        return out


def read_profile_line(path, key, kernel, conv=float):
    """`<key> <kernel> <value>` from a committed counter summary, or None."""
    try:
        with open(path) as fh:
            for ln in fh:
                m = re.match(r"\s*" + key + r"\s+(\S+)\s+(\S+)\s*$", ln)
                if m and m.group(1) == kernel:
                    return conv(m.group(2))
    except OSError:
        pass
    return None


# ---------------------------------------------------------------- CPU baselines (the oracle)
def cpu_baselines(budget_s, eta, compiled=False):
    import torch
    from oracle import ttt_layer_oracle as LO
    from oracle import ttt_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)

    def timed(once, tokens):
        once()  # warm-up
        times = []
        t_end = time.perf_counter() + budget_s
        while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
            t0 = time.perf_counter()
            once()
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        return round(tokens / med, 1), len(times), med

    def op_case(kind, Bn, H_, NC_, F_, FF_, G, grad, mini_batch=None):
        d = make_inputs(torch, Bn, H_, NC_, F_, FF_, seed=7, dtype=torch.float32, eta="dense")
        names = ["XK", "XQ", "XV", "eta", "ln_w", "ln_b", "W1", "b1"] + (["W2", "b2"] if FF_ else [])
        fn = O.ttt_mlp if FF_ else O.ttt_linear

        def once():
            if grad:
                a = {n: d[n].float().requires_grad_(True) for n in names}
                out = fn(*[a[n] for n in names], G, mini_batch=mini_batch)
                out.backward(d["dOut"].float().permute(0, 2, 3, 1, 4))
            else:
                with torch.no_grad():
                    fn(*[d[n].float() for n in names], G, mini_batch=mini_batch)
        return once

    res = {}
    cases = [
        ("c0", "ttt_linear forward, fp32, B=2 H=4 T=256 F=64 (the whole config)",
         op_case("linear", 2, 4, 16, 64, 0, 16, False), 2 * 256),
        ("c1", "ttt_mlp forward, fp32, B=1 H=12 T=2048 F=64 FF=256 (1/8 of the batch)",
         op_case("mlp", 1, H, NC, F, FF, G_MLP, False), T),
        ("c2", "ttt_linear forward + autograd backward, fp32, B=1 H=12 T=2048 F=64 G=16 (1/16 of the batch)",
         op_case("linear", 1, H, NC, F, 0, G_LIN, True), T),
        ("c3", "ttt_mlp forward + autograd backward, fp32, B=1 H=12 T=2048 F=64 FF=256 G=8 (1/16 of the batch)",
         op_case("mlp", 1, H, NC, F, FF, G_MLP, True), T),
    ]
    for key, sample, once, tokens in cases:
        print(f"[bench] CPU baseline {key}", file=sys.stderr, flush=True)
        v, n, med = timed(once, tokens)
        res[key] = {"value": v, "unit": "tokens/s", "cores": cores, "kind": "port",
                    "sample": f"oracle {sample}, median of {n} runs, {med:.3f} s each"}

    if compiled:
        # the same c3 sample with the mini-batch step compiled by inductor for
        # the CPU; the first call (tracing and compiling forward and backward)
        # is timed apart and excluded
        print("[bench] CPU baseline c3 under torch.compile (compiling)", file=sys.stderr, flush=True)
        once = op_case("mlp", 1, H, NC, F, FF, G_MLP, True, mini_batch=torch.compile(O.mlp_mini_batch))
        t0 = time.perf_counter()
        once()
        compile_s = time.perf_counter() - t0
        v, n, med = timed(once, T)
        res["c3_compiled"] = {
            "value": v, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"oracle ttt_mlp forward + autograd backward with its mini-batch step under torch.compile "
                      f"(inductor, CPU), fp32, B=1 H=12 T=2048 F=64 FF=256 G=8 (1/16 of the batch), median of "
                      f"{n} runs, {med:.3f} s each; first call with compilation {compile_s:.0f} s, excluded"}

    # the forecaster's training step (forward + backward) on 2 of the 32 windows
    print("[bench] CPU baseline c4", file=sys.stderr, flush=True)
    cfg, model, x, y = forecaster_setup(torch, 2)
    sd0 = {k: v.detach().float() for k, v in model.state_dict().items()}

    def once4():
        sd = {k: v.clone().requires_grad_(True) for k, v in sd0.items()}
        pred = LO.forecaster_forward(sd, x.float(), cfg, FC_PRED, FC_CH)
        torch.nn.functional.mse_loss(pred, y.float()).backward()
    v, n, med = timed(once4, 2 * FC_L)
    res["c4"] = {"value": v, "unit": "tokens/s", "cores": cores, "kind": "port",
                 "sample": f"oracle forecaster forward + autograd backward, fp32, 2 windows of {FC_L} "
                           f"(1/16 of batch {FC_B}), H={FC_H} F={FC_F} memo M={FC_M}, median of {n} runs, "
                           f"{med:.3f} s each"}
    return res


# ---------------------------------------------------------------- GPU legs
def run_mlp(torch, steps, warmup, eta, only=None, Bn=B, memo=0, fwd_only=False, ckpt=True):
    from ttt_amd.mlp import mlp_backward, mlp_forward
    dev = torch.device("cuda:0")
    g = {k: v.to(dev) for k, v in make_inputs(torch, Bn, H, NC, F, FF, seed=3, eta=eta).items()}
    keys = ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK", "eta")
    rule = "causal" if eta == "lr" else "dense"

    def fwd():
        out, ck, _, last, saved = mlp_forward(*(g[k] for k in keys), G_MLP, M=memo, want_ckpt=ckpt,
                                              want_last=not fwd_only, want_saved=not fwd_only,
                                              ckpt_w1_only=True, eta_rule=rule)
        return out, (ck, last, saved)

    def bwd(saved):
        return mlp_backward(g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], *saved, g["dOut"], G_MLP,
                            eta_rule=rule)

    _, ck = fwd()
    for _ in range(warmup):
        _, ck = fwd()
        if not fwd_only:
            bwd(ck)
    torch.cuda.synchronize()
    tm = Timer(torch)
    t0 = time.perf_counter()
    for _ in range(steps):
        if only != "mlp_bwd":
            tm.mark("ttt_mlp_fwd")
            _, ck = fwd()
        if only != "mlp_fwd" and not fwd_only:
            tm.mark("ttt_mlp_bwd")
            bwd(ck)
    tm.mark(None)
    sp = tm.spans()
    wall = time.perf_counter() - t0
    total = sum(sum(v) for v in sp.values())
    return {k: statistics.mean(v) for k, v in sp.items()}, total, wall


def run_linear(torch, steps, warmup, eta, only=None, Bn=B, H_=H, NC_=NC, dtype=None, fwd_only=False):
    from ttt_amd.linear import linear_backward, linear_forward
    dev = torch.device("cuda:0")
    g = {k: v.to(dev) for k, v in make_inputs(torch, Bn, H_, NC_, F, seed=2, dtype=dtype, eta=eta).items()}
    keys = ("ln_w", "ln_b", "W1", "b1", "XQ", "XV", "XK", "eta")
    rule = "causal" if eta == "lr" else "dense"

    def fwd():
        out, ck, last, saved = linear_forward(*(g[k] for k in keys), min(G_LIN, NC_), want_ckpt=not fwd_only,
                                              want_last=not fwd_only, want_saved=not fwd_only, eta_rule=rule)
        return out, (ck, last, saved)

    def bwd(st):
        ck, last, saved = st
        return linear_backward(g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], ck[0], last[0], saved,
                               g["dOut"], min(G_LIN, NC_), eta_rule=rule)

    _, ck = fwd()
    for _ in range(warmup):
        _, ck = fwd()
        if not fwd_only:
            bwd(ck)
    torch.cuda.synchronize()
    tm = Timer(torch)
    for _ in range(steps):
        if only != "linear_bwd":
            tm.mark("ttt_linear_fwd")
            _, ck = fwd()
        if only != "linear_fwd" and not fwd_only:
            tm.mark("ttt_linear_bwd")
            bwd(ck)
    tm.mark(None)
    sp = tm.spans()
    return {k: statistics.mean(v) for k, v in sp.items()}, sum(sum(v) for v in sp.values())


def run_readout(torch, steps, warmup):
    from ttt_amd.mlp import mlp_cached_readout
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(4)
    xq = torch.randn(B, H, NC, K, F, generator=gen).to(torch.bfloat16).to(dev)
    ws = [0.02 * torch.randn(B, H, F, FF, generator=gen), torch.zeros(B, H, 1, FF),
          0.02 * torch.randn(B, H, FF, F, generator=gen), torch.zeros(B, H, 1, F)]
    ws = [w.to(dev) for w in ws]
    lw, lb = torch.ones(H, F, device=dev), torch.zeros(H, F, device=dev)
    for _ in range(warmup):
        mlp_cached_readout(xq, *ws, lw, lb)
    torch.cuda.synchronize()
    tm = Timer(torch)
    for _ in range(steps):
        tm.mark("ttt_mlp_cached_readout")
        mlp_cached_readout(xq, *ws, lw, lb)
    tm.mark(None)
    sp = tm.spans()
    return statistics.mean(sp["ttt_mlp_cached_readout"])


def memo_pairs(M=MEMO_M):
    """(token, memo state) pairs the combiner evaluates per chain: tokens of
    segment i use the i states before it."""
    NS = math.ceil(NC / M)
    return sum(i * (min((i + 1) * M, NC) - i * M) * K for i in range(NS))


def run_memo(torch, steps, warmup, only=None):
    from ttt_amd.memo import memo_combine_backward, memo_combine_forward
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(5)
    NS = math.ceil(NC / MEMO_M)
    act = [torch.randn(B, H, NC, K, F, generator=gen).to(torch.bfloat16).to(dev) for _ in range(5)]
    xq, xk, xu, xqw, dout = act
    xu = (0.3 * xu.float()).to(torch.bfloat16)
    ws = [0.02 * torch.randn(B, H, NS, F, FF, generator=gen), torch.zeros(B, H, NS, 1, FF),
          0.02 * torch.randn(B, H, NS, FF, F, generator=gen), torch.zeros(B, H, NS, 1, F)]
    ws = [w.to(dev) for w in ws]
    lw, lb = torch.ones(H, F, device=dev), torch.zeros(H, F, device=dev)
    _, gates = memo_combine_forward(xq, xk, xu, xqw, *ws, lw, lb, MEMO_M)
    for _ in range(warmup):
        _, gates = memo_combine_forward(xq, xk, xu, xqw, *ws, lw, lb, MEMO_M)
        memo_combine_backward(xq, xu, xqw, *ws, lw, lb, MEMO_M, gates, dout)
    torch.cuda.synchronize()
    tm = Timer(torch)
    for _ in range(steps):
        if only != "memo_bwd":
            tm.mark("ttt_mlp_memo_combine")
            _, gates = memo_combine_forward(xq, xk, xu, xqw, *ws, lw, lb, MEMO_M)
        if only != "memo_fwd":
            tm.mark("ttt_mlp_memo_combine_bwd")
            memo_combine_backward(xq, xu, xqw, *ws, lw, lb, MEMO_M, gates, dout)
        if only is None:
            # the inference form: no backward follows, so no memo-state images
            tm.mark("ttt_mlp_memo_combine_inference")
            memo_combine_forward(xq, xk, xu, xqw, *ws, lw, lb, MEMO_M, images=False)
    tm.mark(None)
    sp = tm.spans()
    return {k: statistics.mean(v) for k, v in sp.items()}


def forecaster_setup(torch, batch, head_dim=FC_F, mini_batch=K):
    """The end-to-end forecaster (random init) and one batch of windows of the
    synthetic ETTh1-shaped series (lookback 512, horizon 96, 7 channels)."""
    from ttt_amd import series
    from ttt_amd.model import ModelConfig, TTTForecaster
    cfg = ModelConfig(seq_len=FC_L, model_dim=FC_H * head_dim, num_heads=FC_H, ssm_layer="ttt_mlp",
                      mini_batch_size=mini_batch, ttt_base_lr=0.05, mem_cache_segment_n_mini_batches=FC_M,
                      scan_checkpoint_group_size=FC_G)
    torch.manual_seed(0)
    model = TTTForecaster(cfg, d_in=FC_CH, d_out=FC_CH, pred_len=FC_PRED)
    data = series.synthetic_series(seed=0)
    x, y = series.batch(data, batch, FC_L, FC_PRED, FC_PRED, seed=1)
    return cfg, model, x, y[:, -FC_PRED:, :]


def run_forecaster(torch, steps, warmup, head_dim=FC_F, mini_batch=K):
    """One AdamW training step (forward, loss, backward, gradient clipping,
    optimizer step; main.py:73-95 with bf16 autocast, no grad scaler needed)
    and one inference forward, at batch 32."""
    dev = torch.device("cuda:0")
    cfg, model, x, y = forecaster_setup(torch, FC_B, head_dim, mini_batch)
    model = model.to(dev)
    x, y = x.to(dev), y.to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=1e-2)

    def train_step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            pred = model(x)
        loss = torch.nn.functional.mse_loss(pred.float(), y)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        return loss

    def infer():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model(x)

    for _ in range(warmup):
        train_step()
        infer()
    torch.cuda.synchronize()
    tm = Timer(torch)
    t0 = time.perf_counter()
    for _ in range(steps):
        tm.mark("train_step")
        loss = train_step()
    tm.mark(None)
    sp = tm.spans()
    wall_train = (time.perf_counter() - t0) / steps
    tm = Timer(torch)
    t0 = time.perf_counter()
    for _ in range(steps):
        tm.mark("inference")
        infer()
    tm.mark(None)
    si = tm.spans()
    wall_inf = (time.perf_counter() - t0) / steps
    return (statistics.mean(sp["train_step"]), statistics.mean(si["inference"]), wall_train, wall_inf,
            float(loss.item()), cfg)


def run_forecaster_graph(torch, steps, warmup, head_dim=FC_F, mini_batch=K):
    """The same training step and inference forward, each captured once in a
    HIP graph (torch.cuda.CUDAGraph; AdamW with capturable state) and timed
    by replays: the launches' host cost leaves the step.  Replays equal eager
    steps bitwise (tests/test_gpu_layer.py checks it at batch 2)."""
    dev = torch.device("cuda:0")
    cfg, model, x, y = forecaster_setup(torch, FC_B, head_dim, mini_batch)
    model = model.to(dev)
    sx, sy = x.to(dev), y.to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=1e-2, capturable=True)

    def train_step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            pred = model(sx)
        loss = torch.nn.functional.mse_loss(pred.float(), sy)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        return loss

    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(max(warmup, 2)):
            opt.zero_grad(set_to_none=True)
            train_step()
    torch.cuda.current_stream().wait_stream(side)
    g_train = torch.cuda.CUDAGraph()
    opt.zero_grad(set_to_none=True)
    with torch.cuda.graph(g_train):
        loss = train_step()
    g_inf = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                model(sx)
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(g_inf):
            model(sx)
    out = []
    for g in (g_train, g_inf):
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        out.append((time.perf_counter() - t0) / steps)
    return out[0], out[1], float(loss.item())


def roofline(kernel, sec, flops, nbytes, mfma_peak):
    """Binding roofline of one kernel: whichever of MFMA and HBM gives the
    longer ideal time for its algorithmic work."""
    t_mfma, t_hbm = flops / mfma_peak, nbytes / HBM_PEAK
    if t_hbm >= t_mfma:
        r = {"bound": "hbm", "achieved": nbytes / sec / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s"}
    else:
        r = {"bound": "mfma", "achieved": flops / sec / 1e12, "peak": mfma_peak / 1e12, "unit": "TFLOP/s"}
    r["frac"] = r["achieved"] / r["peak"]
    r["achieved"] = round(r["achieved"], 2)
    r["frac"] = round(r["frac"], 4)
    r["traffic"] = read_profile_line(TRAFFIC_FILE, "traffic", kernel, int)
    r["mfma_busy"] = read_profile_line(COUNTER_FILE, "mfma_busy", kernel)
    r["kernel"] = kernel
    r["algorithmic"] = {"flops": flops, "bytes": nbytes, "avg_launch_us": round(sec * 1e6, 2),
                        "mfma_frac": round(flops / sec / mfma_peak, 4),
                        "hbm_frac": round(nbytes / sec / HBM_PEAK, 4)}
    return r


def copy_calibration(torch):
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 3}), flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the TTT chains are independent per (batch, head), so a run on "
              "N GPUs is N copies of this one with B/N each plus one gradient all-reduce; multi-GPU runs "
              "are not part of this build.", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from ttt_amd import _lib
    _lib.load()

    if args.copy_calibration:
        copy_calibration(torch)
        return
    if args.only:
        if args.only.startswith("mlp"):
            k, _, _ = run_mlp(torch, args.steps, args.warmup, args.eta, only=args.only)
        elif args.only.startswith("linear"):
            k, _ = run_linear(torch, args.steps, args.warmup, args.eta, only=args.only)
        elif args.only.startswith("memo"):
            k = run_memo(torch, args.steps, args.warmup, only=args.only)
        elif args.only in ("forecaster", "forecaster_ref"):
            ref = args.only == "forecaster_ref"
            hd, mb = (32, 64) if ref else (FC_F, K)
            tr, inf, _, _, _, _ = run_forecaster(torch, args.steps, args.warmup, head_dim=hd, mini_batch=mb)
            gtr, ginf, _ = run_forecaster_graph(torch, args.steps, args.warmup, head_dim=hd, mini_batch=mb)
            k = {"train_step": tr, "inference": inf, "graph_train_step": gtr, "graph_inference": ginf}
        else:
            k = {"ttt_mlp_cached_readout": run_readout(torch, args.steps, args.warmup)}
        print(json.dumps({"only": args.only, "avg_us": {n: round(v * 1e6, 2) for n, v in k.items()}}), flush=True)
        return

    eta = args.eta
    print(f"[bench] TTT-MLP fwd+bwd B{B} H{H} T{T} F{F} FF{FF} G{G_MLP} bf16, eta {eta}: "
          f"{args.warmup} warm-up + {args.steps} timed steps", file=sys.stderr, flush=True)
    kern, total, wall = run_mlp(torch, args.steps, args.warmup, eta)
    step_s = total / args.steps
    value = B * T / step_s
    other = "dense" if eta == "lr" else "lr"
    print(f"[bench] TTT-MLP fwd+bwd, eta {other}", file=sys.stderr, flush=True)
    kern_o, total_o, _ = run_mlp(torch, args.steps, args.warmup, other)

    print("[bench] TTT-Linear fwd+bwd", file=sys.stderr, flush=True)
    lk, ltotal = run_linear(torch, args.steps, args.warmup, eta)
    print("[bench] TTT-MLP forward B8 (no memo, memo M=2)", file=sys.stderr, flush=True)
    c1, c1_total, _ = run_mlp(torch, args.steps, args.warmup, eta, Bn=8, fwd_only=True, ckpt=False)
    c1m, c1m_total, _ = run_mlp(torch, args.steps, args.warmup, eta, Bn=8, memo=2, fwd_only=True, ckpt=False)
    print("[bench] TTT-Linear forward fp32 B2 H4 T256", file=sys.stderr, flush=True)
    c0, c0_total = run_linear(torch, args.steps, args.warmup, eta, Bn=2, H_=4, NC_=16, dtype=torch.float32,
                              fwd_only=True)
    print("[bench] cached readout", file=sys.stderr, flush=True)
    ro = run_readout(torch, args.steps, args.warmup)
    print(f"[bench] memory-cache combiner (M={MEMO_M})", file=sys.stderr, flush=True)
    mk = run_memo(torch, args.steps, args.warmup)
    print("[bench] forecaster train step + inference", file=sys.stderr, flush=True)
    fc_train, fc_inf, fc_wall_train, fc_wall_inf, fc_loss, _ = run_forecaster(torch, args.steps, args.warmup)
    print("[bench] forecaster train step + inference, each one HIP graph", file=sys.stderr, flush=True)
    fg_train, fg_inf, _ = run_forecaster_graph(torch, args.steps, args.warmup)
    print("[bench] forecaster at the reference ModelConfig shape (K=64, F=FF=32)", file=sys.stderr, flush=True)
    rc_train, rc_inf, _, _, rc_loss, _ = run_forecaster(torch, args.steps, args.warmup, head_dim=32, mini_batch=64)
    rcg_train, rcg_inf, _ = run_forecaster_graph(torch, args.steps, args.warmup, head_dim=32, mini_batch=64)

    state = mlp_state_floats()
    kernels = {
        "ttt_mlp_fwd": roofline("ttt_mlp_fwd", kern["ttt_mlp_fwd"], mlp_fwd_flops(),
                                fwd_bytes(state, G_MLP, F * FF, eta), MFMA_PEAK_BF16),
        "ttt_mlp_bwd": roofline("ttt_mlp_bwd", kern["ttt_mlp_bwd"], 2 * mlp_fwd_flops(),
                                bwd_bytes(state, G_MLP, F * FF, eta), MFMA_PEAK_BF16),
        "ttt_linear_fwd": roofline("ttt_linear_fwd", lk["ttt_linear_fwd"], lin_fwd_flops(),
                                   fwd_bytes(lin_state_floats(), G_LIN, lin_state_floats(), eta), MFMA_PEAK_BF16),
        "ttt_linear_bwd": roofline("ttt_linear_bwd", lk["ttt_linear_bwd"], 2 * lin_fwd_flops(),
                                   bwd_bytes(lin_state_floats(), G_LIN, lin_state_floats(), eta), MFMA_PEAK_BF16),
        "ttt_mlp_cached_readout": roofline("ttt_mlp_cached_readout", ro, readout_flops(), readout_bytes(),
                                           MFMA_PEAK_BF16),
    }
    dominant = max(("ttt_mlp_fwd", "ttt_mlp_bwd"), key=lambda n: kern[n])
    roof = dict(kernels[dominant])

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baselines(args.cpu_seconds, eta, compiled=args.cpu_compile)

    c1_flops = mlp_fwd_flops(Bn=8)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "ttt_mlp forward+backward (the launches TritonMLP.apply makes)", "B": B, "H": H,
                   "T": T, "K": K, "F": F, "FF": FF, "checkpoint_group": G_MLP,
                   "eta": ("per-token lr [B,H,NC,K] fp32, causal rule eta[i][j] = lr[j]/(i+1) expanded on chip"
                           if eta == "lr" else "causal [B,H,NC,K,K] bf16"),
                   "activations": "bf16", "state": "fp32", "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": dict(cpu["c3"]) if cpu else None,
        "cpu_baseline_compiled": dict(cpu["c3_compiled"]) if cpu and "c3_compiled" in cpu else None,
        "mfma_frac_fwd_bwd": round(3 * mlp_fwd_flops() / step_s / MFMA_PEAK_BF16, 4),
        "kernels": {n: {"avg_launch_us": r["algorithmic"]["avg_launch_us"], "bound": r["bound"],
                        "frac": r["frac"], "mfma_frac": r["algorithmic"]["mfma_frac"],
                        "hbm_frac": r["algorithmic"]["hbm_frac"], "mfma_busy": r["mfma_busy"]}
                    for n, r in kernels.items()},
        ("mlp_fwd_bwd_eta_" + other): {"value": round(B * T / (total_o / args.steps), 1), "unit": "tokens/s",
                                       "ms_per_step": round(total_o / args.steps * 1e3, 4),
                                       "fwd_us": round(kern_o["ttt_mlp_fwd"] * 1e6, 2),
                                       "bwd_us": round(kern_o["ttt_mlp_bwd"] * 1e6, 2)},
        "configs": {
            "c0_linear_fwd_fp32_B2H4T256": {"us_per_call": round(c0_total / args.steps * 1e6, 2),
                                            "value": round(2 * 256 / (c0_total / args.steps), 1),
                                            "unit": "tokens/s", "cpu_baseline": cpu["c0"] if cpu else None},
            "c1_mlp_fwd_B8": {"value": round(8 * T / (c1_total / args.steps), 1), "unit": "tokens/s",
                              "us_per_call": round(c1_total / args.steps * 1e6, 2),
                              "mfma_frac": round(c1_flops / (c1_total / args.steps) / MFMA_PEAK_BF16, 4),
                              "with_memo_M2": {"value": round(8 * T / (c1m_total / args.steps), 1),
                                               "us_per_call": round(c1m_total / args.steps * 1e6, 2)},
                              "cpu_baseline": cpu["c1"] if cpu else None},
            "c2_linear_fwd_bwd": {"value": round(B * T / (ltotal / args.steps), 1), "unit": "tokens/s",
                                  "ms_per_step": round(ltotal / args.steps * 1e3, 4), "checkpoint_group": G_LIN,
                                  "hbm_frac_fwd": kernels["ttt_linear_fwd"]["algorithmic"]["hbm_frac"],
                                  "cpu_baseline": cpu["c2"] if cpu else None},
            "c3_mlp_fwd_bwd": {"value": round(value, 1), "unit": "tokens/s", "cpu_baseline": cpu["c3"] if cpu else None},
            "c4_forecaster": {
                "train_step_ms": round(fc_train * 1e3, 3), "train_tokens_per_s": round(FC_B * FC_L / fc_train, 1),
                "inference_ms": round(fc_inf * 1e3, 3), "inference_tokens_per_s": round(FC_B * FC_L / fc_inf, 1),
                "wall_ms_train": round(fc_wall_train * 1e3, 3), "wall_ms_inference": round(fc_wall_inf * 1e3, 3),
                "graph_train_step_ms": round(fg_train * 1e3, 3), "graph_train_tokens_per_s": round(FC_B * FC_L / fg_train, 1),
                "graph_inference_ms": round(fg_inf * 1e3, 3), "graph_inference_tokens_per_s": round(FC_B * FC_L / fg_inf, 1),
                "loss": round(fc_loss, 5),
                "shape": f"batch {FC_B}, lookback {FC_L}, horizon {FC_PRED}, {FC_CH} channels, TTT-MLP H={FC_H} "
                         f"F={FC_F} (model_dim {FC_H * FC_F}), K={K}, memo M={FC_M}, G={FC_G}, bf16 autocast, AdamW",
                "cpu_baseline": cpu["c4"] if cpu else None},
            "forecaster_reference_model_shape": {
                "train_step_ms": round(rc_train * 1e3, 3), "train_tokens_per_s": round(FC_B * FC_L / rc_train, 1),
                "inference_ms": round(rc_inf * 1e3, 3), "inference_tokens_per_s": round(FC_B * FC_L / rc_inf, 1),
                "graph_train_step_ms": round(rcg_train * 1e3, 3),
                "graph_train_tokens_per_s": round(FC_B * FC_L / rcg_train, 1),
                "graph_inference_ms": round(rcg_inf * 1e3, 3),
                "graph_inference_tokens_per_s": round(FC_B * FC_L / rcg_inf, 1),
                "loss": round(rc_loss, 5),
                "shape": f"as c4 with ModelConfig's defaults of main.py: model_dim 128 over H={FC_H} heads (F=32, "
                         f"FF=32), K=64 (the register-resident one-wave kernels), memo M={FC_M}, G={FC_G}"},
        },
        "memo_combine": {
            "value": round(B * T / (mk["ttt_mlp_memo_combine"] + mk["ttt_mlp_memo_combine_bwd"]), 1),
            "unit": "tokens/s", "fwd_ms": round(mk["ttt_mlp_memo_combine"] * 1e3, 4),
            "bwd_ms": round(mk["ttt_mlp_memo_combine_bwd"] * 1e3, 4),
            "inference_fwd_ms": round(mk["ttt_mlp_memo_combine_inference"] * 1e3, 4), "memo_segment": MEMO_M,
            "readouts_per_chain": memo_pairs(),
            "mfma_frac_fwd": round(4 * F * FF * memo_pairs() * B * H / mk["ttt_mlp_memo_combine"] / MFMA_PEAK_BF16, 4),
            "shape": f"B{B} H{H} T{T} F{F} FF{FF}, {math.ceil(NC / MEMO_M)} memo states per chain, bf16"},
        "cached_readout": {"value": round(B * T / ro, 1), "unit": "tokens/s",
                           "ms_per_launch": round(ro * 1e3, 4),
                           "shape": f"XQ [{B},{H},{NC},{K},{F}] bf16, one fixed state per chain"},
        "wall_s_mlp_timed": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
