"""Writes tests/golden/trained_forecaster_etth1.safetensors: the reference's
trained forecaster (ttt_forecaster.pt, written by main.py:107 after 20 epochs
on ETTh1) and eight validation windows of the series it was trained on.

Run in a container that holds the reference at /root/reference:

    python tests/golden/make_trained_forecaster.py

The checkpoint is read with torch.load(weights_only=True) (plain tensors, no
code).  The windows restate Dataset_ETT_hour (data_loader.py:43-99) for
main.py's settings (features "S": the OT column alone; seq_len 384, label_len
96, pred_len 96): a StandardScaler fitted on the first 12*30*24 rows (the
training split), the validation split starting 384 rows before row 8640, and
for window i the input rows [i, i + 384) and the target rows [i + 384, i + 480)
of that split (main.py:82 keeps the last pred_len rows of batch_y).
"""

from __future__ import annotations

import os

import numpy as np
import pandas as pd
import torch
from safetensors.torch import save_file

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "trained_forecaster_etth1.safetensors")

SEQ_LEN, PRED_LEN = 384, 96
TRAIN_END = 12 * 30 * 24               # data_loader.py:48 (border2s[0])
VAL_BEGIN = TRAIN_END - SEQ_LEN        # border1s[1], data_loader.py:47
VAL_END = TRAIN_END + 4 * 30 * 24      # border2s[1]
N_WINDOWS = 8


def main() -> None:
    sd = torch.load(os.path.join(REF, "ttt_forecaster.pt"), map_location="cpu", weights_only=True)
    ot = pd.read_csv(os.path.join(REF, "ETT", "ETTh1.csv"))["OT"].to_numpy(dtype=np.float64)
    train = ot[:TRAIN_END]
    mean, std = train.mean(), train.std()   # StandardScaler: population std
    series = (ot - mean) / std
    val = series[VAL_BEGIN:VAL_END]
    n_val = len(val) - SEQ_LEN - PRED_LEN + 1  # Dataset_ETT_hour.__len__
    idx = np.linspace(0, n_val - 1, N_WINDOWS).round().astype(np.int64)
    x = np.stack([val[i:i + SEQ_LEN] for i in idx])[..., None]
    y = np.stack([val[i + SEQ_LEN:i + SEQ_LEN + PRED_LEN] for i in idx])[..., None]
    tensors = {k: v.contiguous() for k, v in sd.items()}
    tensors["x"] = torch.from_numpy(x).float().contiguous()
    tensors["y"] = torch.from_numpy(y).float().contiguous()
    tensors["window_index"] = torch.from_numpy(idx)
    tensors["scaler_mean_std"] = torch.tensor([mean, std], dtype=torch.float64)
    save_file(tensors, OUT, metadata={
        "source": "reference ttt_forecaster.pt (main.py) and ETTh1.csv validation windows",
        "config": "seq_len 384, model_dim 128, num_heads 4, ttt_mlp, mini_batch 64, base lr 0.05, "
                  "checkpoint group 16, d_in 1, d_out 1, pred_len 96"})
    print(f"wrote {OUT}: {len(sd)} parameters, windows {idx.tolist()}")


if __name__ == "__main__":
    main()
