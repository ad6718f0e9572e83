"""The reference's trained forecaster (ttt_forecaster.pt from main.py, kept as
tests/golden/trained_forecaster_etth1.safetensors with eight ETTh1
validation windows; tests/golden/make_trained_forecaster.py writes it).

CPU checks: the checkpoint loads strictly into TTTForecaster at main.py's
configuration, the fixture holds the checkpoint bit for bit (when the
reference is present), and the windows are the restated Dataset_ETT_hour
windows (standardised with the training split's statistics).  The GPU
inference and gradients on these weights are in tests/test_gpu_trained.py."""

import os

import pytest
import torch

from tests._trained import FIXTURE, REF_CKPT, main_config, trained

safetensors = pytest.importorskip("safetensors")


def test_fixture_loads_strictly_into_the_forecaster():
    from ttt_amd.model import TTTForecaster
    sd, x, y = trained()
    model = TTTForecaster(main_config(), d_in=1, d_out=1, pred_len=96)
    res = model.load_state_dict(sd, strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    assert x.shape == (8, 384, 1) and y.shape == (8, 96, 1)
    assert x.dtype == torch.float32 and y.dtype == torch.float32


@pytest.mark.skipif(not os.path.exists(REF_CKPT), reason="the reference checkpoint is not in this container")
def test_fixture_is_the_reference_checkpoint():
    ref = torch.load(REF_CKPT, map_location="cpu", weights_only=True)
    sd, _, _ = trained()
    assert set(ref) == set(sd)
    for k, v in ref.items():
        assert torch.equal(v, sd[k]), k


def test_windows_are_standardised_validation_windows():
    """The windows come from the validation split, standardised by the
    training split's mean and population std: the input of window i + 1
    starts later in the same series, and targets continue the inputs' series
    (window 0's input tail and target of a later window overlap exactly where
    their row ranges do)."""
    from safetensors.torch import load_file
    t = load_file(FIXTURE)
    idx = t["window_index"].tolist()
    x, y = t["x"][..., 0].double(), t["y"][..., 0].double()
    assert idx == sorted(idx) and idx[0] == 0
    mean, std = t["scaler_mean_std"].tolist()
    assert std > 0
    # two windows whose row ranges overlap agree on the shared rows
    for a, b in zip(range(len(idx) - 1), range(1, len(idx))):
        da, db = idx[a], idx[b]
        if db - da < 384:
            assert torch.equal(x[a, db - da:], x[b, :384 - (db - da)])
    # every value lies in the standardised series' plausible range
    assert float(x.abs().max()) < 10 and float(y.abs().max()) < 10
