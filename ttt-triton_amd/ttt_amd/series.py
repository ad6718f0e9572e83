"""Synthetic ETTh1-shaped series and forecasting windows for the end-to-end
forecaster workload (no dataset is available offline).

The series has the shape of ETT/ETTh1.csv (7 channels x 17420 hourly steps
from 2016-07-01 00:00): each channel is a 24-step and a 168-step sinusoid
with amplitudes U(0.5, 2) and random phases, plus a linear drift and AR(1)
noise (phi = 0.9, sigma = 0.3), then standardised per channel with the
statistics of the training split, as Dataset_ETT_hour does with its
StandardScaler (data_loader.py:44-61; splits of 12/4/4 months of 30 days,
data_loader.py:47-48).  Time features are the four hourly ones of
util/timefeatures.py:106 (hour of day, day of week, day of month, day of
year, each scaled to [-0.5, 0.5]).  Windows follow
Dataset_ETT_hour.__getitem__ (data_loader.py:85-99)."""

from __future__ import annotations

import datetime as _dt

import numpy as np
import torch

N_STEPS, N_CHANNELS = 17420, 7
TRAIN_END = 12 * 30 * 24


def synthetic_series(n_steps: int = N_STEPS, n_channels: int = N_CHANNELS, seed: int = 0) -> np.ndarray:
    """[n_steps, n_channels] float32, standardised with the training split's
    per-channel mean and (biased) std."""
    rng = np.random.default_rng(seed)
    t = np.arange(n_steps, dtype=np.float64)
    out = np.empty((n_steps, n_channels), dtype=np.float64)
    for c in range(n_channels):
        a1, a2 = rng.uniform(0.5, 2.0, size=2)
        p1, p2 = rng.uniform(0.0, 2 * np.pi, size=2)
        drift = rng.normal(0.0, 1.0) / n_steps
        eps = rng.normal(0.0, 0.3, size=n_steps)
        ar = np.empty(n_steps)
        acc = 0.0
        for i in range(n_steps):
            acc = 0.9 * acc + eps[i]
            ar[i] = acc
        out[:, c] = a1 * np.sin(2 * np.pi * t / 24 + p1) + a2 * np.sin(2 * np.pi * t / 168 + p2) + drift * t + ar
    train = out[:min(TRAIN_END, n_steps)]
    mu, sd = train.mean(0), train.std(0)
    return ((out - mu) / np.where(sd > 0, sd, 1.0)).astype(np.float32)


def time_features(n_steps: int, start=_dt.datetime(2016, 7, 1)) -> np.ndarray:
    """[n_steps, 4] float32: hour/23, weekday/6, (day-1)/30, (yday-1)/365, each minus 0.5."""
    rows = []
    for i in range(n_steps):
        d = start + _dt.timedelta(hours=i)
        rows.append((d.hour / 23.0 - 0.5, d.weekday() / 6.0 - 0.5, (d.day - 1) / 30.0 - 0.5,
                     (d.timetuple().tm_yday - 1) / 365.0 - 0.5))
    return np.asarray(rows, dtype=np.float32)


def split_bounds(flag: str, seq_len: int):
    """(start, end) of a split, data_loader.py:47-48 (12/4/4 months of 30 days)."""
    b1 = [0, TRAIN_END - seq_len, TRAIN_END + 4 * 30 * 24 - seq_len]
    b2 = [TRAIN_END, TRAIN_END + 4 * 30 * 24, TRAIN_END + 8 * 30 * 24]
    i = {"train": 0, "val": 1, "test": 2}[flag]
    return b1[i], b2[i]


def windows(series: np.ndarray, index: np.ndarray, seq_len: int, label_len: int, pred_len: int):
    """(seq_x [N, seq_len, C], seq_y [N, label_len + pred_len, C]) for window
    starts `index` into `series` (data_loader.py:85-99)."""
    idx = np.asarray(index)
    xs = np.stack([series[s:s + seq_len] for s in idx])
    ys = np.stack([series[s + seq_len - label_len:s + seq_len + pred_len] for s in idx])
    return torch.from_numpy(xs), torch.from_numpy(ys)


def batch(series: np.ndarray, batch_size: int, seq_len: int, label_len: int, pred_len: int, flag: str = "train",
          seed: int = 0):
    """One batch of windows drawn (seeded) from a split."""
    lo, hi = split_bounds(flag, seq_len)
    n = (hi - lo) - seq_len - pred_len + 1
    rng = np.random.default_rng(seed)
    return windows(series[lo:hi], rng.integers(0, n, size=batch_size), seq_len, label_len, pred_len)


__all__ = ["synthetic_series", "time_features", "split_bounds", "windows", "batch", "N_STEPS", "N_CHANNELS"]
