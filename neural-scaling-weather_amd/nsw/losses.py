"""Latitude-weighted RMSE (utils/losses.py:230-266) and ACC on libnsw.

``WeightedRMSE`` keeps the reference's constructor and forward signature.
The reduction is one libnsw kernel pass over pred and target computing, per
(b, t, c) plane, the float64 sums the reference ends up with (fp32 difference
and square times the float64 cos-lat weights); the means over batch / time are
applied to the [B, T, C] result.  ``WeightedACC`` is the textbook
latitude-weighted anomaly correlation (no counterpart in the reference).
"""
from __future__ import annotations

import torch
from torch import nn

from . import torch_ops  # noqa: F401  (registers torch.ops.nsw.*)


def _reduce_leading(v: torch.Tensor, temporal_average: bool) -> torch.Tensor:
    # utils/losses.py:259-264: mean over b (and over t while dims > 1)
    if temporal_average:
        while v.dim() > 1:
            v = v.mean(dim=0)
        return v
    return v.mean(dim=0)


def _out_dtype(weights: torch.Tensor, pred: torch.Tensor) -> torch.dtype:
    return torch.promote_types(weights.dtype, pred.dtype)


class WeightedRMSE(nn.Module):
    """Weighted RMSE function"""

    def __init__(self, weights: torch.Tensor = None, temporal_average: bool = True):
        super().__init__()
        assert weights is not None, "Weights needed!"
        self.temporal_average = temporal_average
        self.register_buffer("weights", weights)

    def forward(self, pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        w = self.weights
        rmse, _ = torch.ops.nsw.weighted_metrics(pred, target, w, None)
        return _reduce_leading(rmse.to(_out_dtype(w, pred)), self.temporal_average)


class WeightedACC(nn.Module):
    """Latitude-weighted anomaly correlation coefficient against a per-channel
    climatology: acc = sum w af ao / sqrt(sum w af^2 * sum w ao^2)."""

    def __init__(self, weights: torch.Tensor = None, climatology: torch.Tensor = None,
                 temporal_average: bool = True):
        super().__init__()
        assert weights is not None and climatology is not None, "Weights and climatology needed!"
        self.temporal_average = temporal_average
        self.register_buffer("weights", weights)
        self.register_buffer("climatology", climatology)

    def forward(self, pred: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        _, acc = torch.ops.nsw.weighted_metrics(pred, target, self.weights, self.climatology)
        return _reduce_leading(acc.to(_out_dtype(self.weights, pred)), self.temporal_average)


def weighted_rmse_acc(pred, target, weights, climatology=None, temporal_average: bool = True):
    """Both metrics from one pass over the fields."""
    rmse, acc = torch.ops.nsw.weighted_metrics(pred, target, weights, climatology)
    dt = _out_dtype(weights, pred)
    r = _reduce_leading(rmse.to(dt), temporal_average)
    a = None if climatology is None else _reduce_leading(acc.to(dt), temporal_average)
    return r, a
