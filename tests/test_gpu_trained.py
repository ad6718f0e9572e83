"""The forecaster on the reference's trained weights (main.py's checkpoint,
tests/golden/trained_forecaster_etth1.safetensors) and eight ETTh1
validation windows, against the fp64 oracle (oracle/ttt_layer_oracle.py) on
the same weights and windows: trained weights and real data give the
kernels magnitudes random initialisation does not (a trained lr gate, W1/W2
and LayerNorm parameters far from their initial values).

Tolerances: fp32 rel-L2 within max(1e-4, C_FP32 times the fp32 oracle's
own rel-L2 error against fp64); bf16 and fp16 autocast rel-L2 2e-2, with the
norm floors of tests/test_gpu_layer.py for tiny parameter gradients and a
looser one for vanishing ones (below)."""

import sys

import pytest
import torch

from oracle import ttt_layer_oracle as LO
from tests._trained import main_config, trained
from tests._util import C_FP32, rel_l2

pytestmark = pytest.mark.gpu

RTOL_16 = 2e-2
FP32_RTOL = 1e-4
TINY, RTOL_16_TINY = 1e-2, 0.25
# 16-bit bar for a gradient below VANISHING times the largest one: on the
# trained weights the XU projection's gradient is 4e-6 of the largest (the
# output bias's), formed only through the memory-cache gates, i.e. by
# differences between readouts of nearly equal memo states, each taken with
# 16-bit operands as the reference's readout takes them
# (kernels/mlp_cached_readout.py:97-101).  Measured in bf16: 0.35.
VANISHING, RTOL_16_VANISHING = 1e-4, 0.5


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _model(sd):
    from ttt_amd.model import TTTForecaster
    m = TTTForecaster(main_config(), d_in=1, d_out=1, pred_len=96)
    m.load_state_dict(sd, strict=True)
    return m.cuda()


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
def test_trained_inference_vs_oracle(dt):
    sd, x, _ = trained()
    cfg = main_config()
    _say(f"trained forecaster inference {dt}")
    ref = LO.forecaster_forward({k: v.double() for k, v in sd.items()}, x.double(), cfg, 96, 1)
    model = _model(sd).eval()
    with torch.no_grad(), torch.autocast("cuda", dtype=dt, enabled=dt != torch.float32):
        out = model(x.cuda())
    torch.cuda.synchronize()
    err = rel_l2(out.float(), ref)
    if dt == torch.float32:
        ref32 = LO.forecaster_forward({k: v.float() for k, v in sd.items()}, x.float(), cfg, 96, 1)
        bound = max(FP32_RTOL, C_FP32 * rel_l2(ref32, ref))
    else:
        bound = RTOL_16
    _say(f"  prediction rel-L2 {err:.3e} (bound {bound:.3e})")
    assert err <= bound


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_trained_train_step_vs_oracle(dt):
    """One training step's loss and every parameter gradient on the trained
    weights (MSE against the windows' targets, as main.py:88-89 trains)."""
    sd, x, y = trained()
    cfg = main_config()
    _say(f"trained forecaster train step {dt}")
    ref_sd = {k: v.double().requires_grad_(True) for k, v in sd.items()}
    loss_ref = torch.nn.functional.mse_loss(LO.forecaster_forward(ref_sd, x.double(), cfg, 96, 1), y.double())
    loss_ref.backward()
    rtol32 = {}
    if dt == torch.float32:
        sd32 = {k: v.float().requires_grad_(True) for k, v in sd.items()}
        torch.nn.functional.mse_loss(LO.forecaster_forward(sd32, x.float(), cfg, 96, 1), y.float()).backward()
        rtol32 = {k: rel_l2(sd32[k].grad, ref_sd[k].grad) for k in sd}
    model = _model(sd)
    with torch.autocast("cuda", dtype=dt, enabled=dt != torch.float32):
        out = model(x.cuda())
    loss = torch.nn.functional.mse_loss(out.float(), y.cuda())
    loss.backward()
    torch.cuda.synchronize()
    tol = FP32_RTOL if dt == torch.float32 else RTOL_16
    err = abs(loss.item() - loss_ref.item()) / abs(loss_ref.item())
    _say(f"  loss {loss.item():.6f} vs {loss_ref.item():.6f}: rel {err:.3e}")
    bad = ["loss"] if err > tol else []
    gmax = max(float(g.grad.norm()) for g in ref_sd.values())
    for name, prm in model.named_parameters():
        r = ref_sd[name].grad
        e = rel_l2(prm.grad, r)
        if dt == torch.float32:
            tp = max(tol, C_FP32 * rtol32[name])
        elif float(r.norm()) < VANISHING * gmax:
            tp = RTOL_16_VANISHING
        else:
            tp = RTOL_16_TINY if float(r.norm()) < TINY * gmax else tol
        _say(f"  d{name}: rel-L2 {e:.3e} (|ref| {float(r.norm()):.3e}), bound ratio {e / tp:.2f}")
        if e > tp:
            bad.append(name)
    assert not bad
