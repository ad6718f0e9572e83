"""Throughput of the TTT-MLP / TTT-Linear inner loop on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]

Headline workload: TTT-MLP forward+backward, B=16, H=12, T=2048 (NC=128
mini-batches of K=16), F=64, hidden 256, bf16 activations, fp32 fast-weight
state, checkpoints every G=8 mini-batches, causal eta.  One step = the
forward kernel (writing the checkpoints) + the backward kernel, through the
same launchers TritonMLP.apply uses, on synthetic seeded inputs already
resident in HBM.  The line also carries TTT-Linear forward+backward (same
B/H/T/F, G=16) and the cached readout of the whole sequence against one fixed
state, each timed the same way.

Every kernel launch is bracketed by HIP events on the stream it runs on, so
the per-kernel averages behind `roofline` come from the timed steps.
`roofline.traffic` (HBM bytes per launch) is read from the committed
rocprofv3 counter summary when it exists for this workload.

The CPU baseline times the oracle (eager PyTorch restatement of the
reference's ops path, fp32, autograd for the backward) on one batch row
(B=1, all 12 heads, all 2048 tokens) on this host's cores.

Other modes (for counter collection):
    --only mlp_fwd|mlp_bwd|linear_fwd|linear_bwd|readout|memo_fwd|memo_bwd   run that kernel alone

The memory-cache combiner (the segment loop of TTTMLP.ttt) is timed at the
same B/H/T/F/FF with memo segments of MEMO_M mini-batches, on synthetic memo
states, forward and backward.
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

B, H, T, K, F, FF = 16, 12, 2048, 16, 64, 256
NC = T // K
G_MLP, G_LIN = 8, 16
MEMO_M = 8  # memo segment size (mini-batches) of the combiner leg


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    ap.add_argument("--only", choices=["mlp_fwd", "mlp_bwd", "linear_fwd", "linear_bwd", "readout", "memo_fwd",
                                       "memo_bwd"])
    ap.add_argument("--copy-calibration", action="store_true")
    return ap.parse_args()


# ---------------------------------------------------------------- algorithmic counts
def mlp_state_floats():
    return 2 * F * FF + FF + F


def lin_state_floats():
    return F * F + F


def mlp_fwd_flops():
    return (14 * F * FF + 6 * K * FF + 6 * K * F) * B * H * T


def lin_fwd_flops():
    return (6 * F * F + 6 * K * F) * B * H * T


def fwd_bytes(state, G, ckpt, sx=2, seta=2):
    """inputs XQ, XK, XV, eta read + out written + state read/written + checkpoints
    written (`ckpt` floats each: what the backward reads of the state)"""
    return (B * H * T * (3 * F * sx + K * seta + F * sx) + B * H * state * 4 * 2
            + B * H * math.ceil(NC / G) * ckpt * 4)


def bwd_bytes(state, G, ckpt, sx=2, seta=2):
    """XQ, XK, XV, dout, eta read + dXQ, dXK, dXV, deta written + checkpoints read
    + state gradients written (and the per-chain LN partials)"""
    return (B * H * T * (4 * F * sx + K * seta) + B * H * T * (3 * F * sx + K * seta)
            + B * H * math.ceil(NC / G) * ckpt * 4 + B * H * (state + 2 * F) * 4 * 2)


def readout_flops():
    return 4 * F * FF * B * H * T


def readout_bytes(sx=2):
    return B * H * T * F * (sx + 4) + B * H * mlp_state_floats() * 4


# ---------------------------------------------------------------- inputs
def make_mlp_inputs(dev, torch, O):
    d = O.make_inputs(B, H, NC, K, F, FF=FF, seed=3, dtype=torch.bfloat16, with_grad=True)
    return {k: v.to(dev) for k, v in d.items()}


def make_lin_inputs(dev, torch, O):
    d = O.make_inputs(B, H, NC, K, F, seed=2, dtype=torch.bfloat16, with_grad=True)
    return {k: v.to(dev) for k, v in d.items()}


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


def read_traffic(kernel):
    """HBM bytes per launch for `kernel` on this workload from the committed
    counter summary (a line `traffic <kernel> <bytes>`), or None."""
    try:
        with open(TRAFFIC_FILE) as fh:
            for ln in fh:
                m = re.match(r"\s*traffic\s+(\S+)\s+(\d+)\s*$", ln)
                if m and m.group(1) == kernel:
                    return int(m.group(2))
    except OSError:
        pass
    return None


# ---------------------------------------------------------------- CPU baseline
def cpu_baseline(budget_s):
    import torch
    from oracle import ttt_oracle as O

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    d = O.make_inputs(1, H, NC, K, F, FF=FF, seed=3, dtype=torch.bfloat16, with_grad=True)
    names = ["XK", "XQ", "XV", "eta", "ln_w", "ln_b", "W1", "b1", "W2", "b2"]

    def once():
        args = {n: d[n].float().requires_grad_(True) for n in names}
        out = O.ttt_mlp(*[args[n] for n in names], G_MLP)
        out.backward(d["dOut"].float().permute(0, 2, 3, 1, 4))

    once()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(T / med, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"oracle ttt_mlp fwd+autograd bwd, fp32, B=1 H=12 T=2048 F=64 FF=256 G=8 "
                      f"(1/16 of the batch), median of {len(times)} runs, {med:.2f} s each"}


# ---------------------------------------------------------------- GPU legs
def run_mlp(torch, O, steps, warmup, only=None):
    from ttt_amd.mlp import mlp_backward, mlp_forward
    dev = torch.device("cuda:0")
    g = make_mlp_inputs(dev, torch, O)
    keys = ("ln_w", "ln_b", "W1", "b1", "W2", "b2", "XQ", "XV", "XK", "eta")

    def fwd():
        out, ck, _, last, saved = mlp_forward(*(g[k] for k in keys), G_MLP, want_ckpt=True, want_last=True,
                                              want_saved=True, ckpt_w1_only=True)
        return out, (ck, last, saved)

    def bwd(saved):
        return mlp_backward(g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], *saved, g["dOut"], G_MLP)

    _, ck = fwd()
    for _ in range(warmup):
        _, ck = fwd()
        bwd(ck)
    torch.cuda.synchronize()
    tm = Timer(torch)
    tm.mark("step")
    t0 = time.perf_counter()
    for _ in range(steps):
        if only != "mlp_bwd":
            tm.mark("ttt_mlp_fwd")
            _, ck = fwd()
        if only != "mlp_fwd":
            tm.mark("ttt_mlp_bwd")
            bwd(ck)
    tm.mark(None)
    sp = tm.spans()
    wall = time.perf_counter() - t0
    total = sum(sum(v) for k, v in sp.items() if k != "step")
    return {k: statistics.mean(v) for k, v in sp.items() if k != "step"}, total, wall


def run_linear(torch, O, steps, warmup, only=None):
    from ttt_amd.linear import linear_backward, linear_forward
    dev = torch.device("cuda:0")
    g = make_lin_inputs(dev, torch, O)
    keys = ("ln_w", "ln_b", "W1", "b1", "XQ", "XV", "XK", "eta")

    def fwd():
        out, ck, last, saved = linear_forward(*(g[k] for k in keys), G_LIN, want_ckpt=True, want_last=True,
                                              want_saved=True)
        return out, (ck[0], last[0], saved)

    def bwd(ck):
        return linear_backward(g["ln_w"], g["ln_b"], g["XQ"], g["XV"], g["XK"], g["eta"], *ck, g["dOut"], G_LIN)

    _, ck = fwd()
    for _ in range(warmup):
        _, ck = fwd()
        bwd(ck)
    torch.cuda.synchronize()
    tm = Timer(torch)
    for _ in range(steps):
        if only != "linear_bwd":
            tm.mark("ttt_linear_fwd")
            _, ck = fwd()
        if only != "linear_fwd":
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
    tm.mark(None)
    sp = tm.spans()
    return {k: statistics.mean(v) for k, v in sp.items()}


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
    r["traffic"] = read_traffic(kernel)
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
    from oracle import ttt_oracle as O

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
            k, _, _ = run_mlp(torch, O, args.steps, args.warmup, only=args.only)
        elif args.only.startswith("linear"):
            k, _ = run_linear(torch, O, args.steps, args.warmup, only=args.only)
        elif args.only.startswith("memo"):
            k = run_memo(torch, args.steps, args.warmup, only=args.only)
        else:
            k = {"ttt_mlp_cached_readout": run_readout(torch, args.steps, args.warmup)}
        print(json.dumps({"only": args.only, "avg_launch_us": {n: round(v * 1e6, 2) for n, v in k.items()}}),
              flush=True)
        return

    print(f"[bench] TTT-MLP fwd+bwd B{B} H{H} T{T} F{F} FF{FF} G{G_MLP} bf16: "
          f"{args.warmup} warm-up + {args.steps} timed steps", file=sys.stderr, flush=True)
    kern, total, wall = run_mlp(torch, O, args.steps, args.warmup)
    step_s = total / args.steps
    value = B * T / step_s

    print("[bench] TTT-Linear fwd+bwd", file=sys.stderr, flush=True)
    lk, ltotal = run_linear(torch, O, args.steps, args.warmup)
    print("[bench] cached readout", file=sys.stderr, flush=True)
    ro = run_readout(torch, args.steps, args.warmup)
    print(f"[bench] memory-cache combiner (M={MEMO_M})", file=sys.stderr, flush=True)
    mk = run_memo(torch, args.steps, args.warmup)

    state = mlp_state_floats()
    kernels = {
        "ttt_mlp_fwd": roofline("ttt_mlp_fwd", kern["ttt_mlp_fwd"], mlp_fwd_flops(), fwd_bytes(state, G_MLP, F * FF),
                                MFMA_PEAK_BF16),
        "ttt_mlp_bwd": roofline("ttt_mlp_bwd", kern["ttt_mlp_bwd"], 2 * mlp_fwd_flops(),
                                bwd_bytes(state, G_MLP, F * FF), MFMA_PEAK_BF16),
        "ttt_linear_fwd": roofline("ttt_linear_fwd", lk["ttt_linear_fwd"], lin_fwd_flops(),
                                   fwd_bytes(lin_state_floats(), G_LIN, lin_state_floats()), MFMA_PEAK_BF16),
        "ttt_linear_bwd": roofline("ttt_linear_bwd", lk["ttt_linear_bwd"], 2 * lin_fwd_flops(),
                                   bwd_bytes(lin_state_floats(), G_LIN, lin_state_floats()), MFMA_PEAK_BF16),
        "ttt_mlp_cached_readout": roofline("ttt_mlp_cached_readout", ro, readout_flops(), readout_bytes(),
                                           MFMA_PEAK_BF16),
    }
    dominant = max(("ttt_mlp_fwd", "ttt_mlp_bwd"), key=lambda n: kern[n])
    roof = {k: v for k, v in kernels[dominant].items()}

    cpu = None
    if not args.no_cpu:
        print(f"[bench] CPU baseline (~{args.cpu_seconds:.0f} s)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.cpu_seconds)

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
        "config": {"workload": "ttt_mlp forward+backward (TritonMLP launchers)", "B": B, "H": H, "T": T,
                   "K": K, "F": F, "FF": FF, "checkpoint_group": G_MLP, "eta": "causal [B,H,NC,K,K]",
                   "activations": "bf16", "state": "fp32", "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "mfma_frac_fwd_bwd": round(3 * mlp_fwd_flops() / step_s / MFMA_PEAK_BF16, 4),
        "kernels": {n: {"avg_launch_us": r["algorithmic"]["avg_launch_us"], "bound": r["bound"],
                        "frac": r["frac"], "mfma_frac": r["algorithmic"]["mfma_frac"],
                        "hbm_frac": r["algorithmic"]["hbm_frac"]} for n, r in kernels.items()},
        "linear_fwd_bwd": {"value": round(B * T / (ltotal / args.steps), 1), "unit": "tokens/s",
                           "ms_per_step": round(ltotal / args.steps * 1e3, 4), "checkpoint_group": G_LIN},
        "memo_combine": {
            "value": round(B * T / (mk["ttt_mlp_memo_combine"] + mk["ttt_mlp_memo_combine_bwd"]), 1),
            "unit": "tokens/s", "fwd_ms": round(mk["ttt_mlp_memo_combine"] * 1e3, 4),
            "bwd_ms": round(mk["ttt_mlp_memo_combine_bwd"] * 1e3, 4), "memo_segment": MEMO_M,
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
