"""Autoregressive forecast of one initial condition with per-step weighted
RMSE / ACC (the loop of utils/inferencer.py:339-449 over lead times, for one
IC and batch 1, without the data loading, spectra and plotting around it).

Per lead step i (utils/inferencer.py:393-449):
    inputs = window with the invariant channels appended
             (preprocessor, mode "inference", utils/data_utils.py:175-197)
    gen    = model(inputs)
    pred   = gen * std + mean,   target_i * std + mean
    rmse_i = WeightedRMSE(pred, target_i) (+ ACC against a climatology)
    window = roll(window, -1, time); window[:, -1] = gen

Here the window is a ring buffer of T frames in fp32 (the dtype of the
reference's input window): the model reads frame t from slot (t + head) mod T
and writes its prediction, converted to fp32, straight into the oldest slot,
which becomes the newest; the invariants enter inside the patch gather;
unnormalisation is fused into the metric reduction.  Nothing is copied or
concatenated per step.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops


class Rollout:
    """Runs ``model`` (a ``nsw.swin.SwinTransformer``) autoregressively.

    mean, std     per-channel normalisation [C] (the inferencer's self.mean /
                  self.std)
    area_weights  latitude weights [H] or [H, 1] (cos-lat / mean), or [H, W]
    invariants    [C_inv, H, W] or None, in the window dtype (fp32)
    clim          per-channel climatology [C] for the ACC, or None
    """

    def __init__(self, model, mean: torch.Tensor, std: torch.Tensor, area_weights: torch.Tensor,
                 invariants: Optional[torch.Tensor] = None, clim: Optional[torch.Tensor] = None):
        self.model = model
        dev = model.head.weight.device
        # the statistics keep their dtype: float64 stats make the reference's
        # unnormalised fields float64 (torch.as_tensor of the stats file,
        # utils/dataloaders/era5hdf5.py:111-122), fp32 stats keep them fp32
        mean, std = torch.as_tensor(mean), torch.as_tensor(std)
        sdt = torch.float64 if torch.float64 in (mean.dtype, std.dtype) else torch.float32
        self.mean = mean.reshape(-1).to(device=dev, dtype=sdt)
        self.std = std.reshape(-1).to(device=dev, dtype=sdt)
        self.weights = area_weights.to(device=dev, dtype=torch.float64)
        self.invariants = None if invariants is None else invariants.to(device=dev, dtype=torch.float32).contiguous()
        self.clim = None if clim is None else clim.reshape(-1).to(device=dev, dtype=torch.float32)

    @torch.no_grad()
    def run(self, input_window: torch.Tensor, targets: torch.Tensor, keep_fields: bool = False):
        """input_window [1, T, C, H, W] (normalised), targets [S, C, H, W]
        (normalised, the truth at lead steps 1..S).  Returns (rmse [S, C],
        acc [S, C] or None, fields [S, C, H, W] fp32 or None) with float64
        metrics on the device."""
        if input_window.dim() != 5 or input_window.shape[0] != 1:
            raise ValueError("input_window must be [1, T, C, H, W]")
        _, T, C, H, W = input_window.shape
        if targets.dim() != 4 or tuple(targets.shape[1:]) != (C, H, W):
            raise ValueError(f"targets must be [S, {C}, {H}, {W}]")
        dev = self.model.head.weight.device
        ring = input_window.to(device=dev, dtype=torch.float32).contiguous().clone()
        tg = targets.to(device=dev, dtype=torch.float32).contiguous()
        S = tg.shape[0]
        rmse = torch.empty(S, C, dtype=torch.float64, device=dev)
        acc = torch.empty(S, C, dtype=torch.float64, device=dev) if self.clim is not None else None
        fields = torch.empty(S, C, H, W, dtype=torch.float32, device=dev) if keep_fields else None
        head = 0                                   # ring slot of model frame 0
        for i in range(S):
            slot = ring[:, head:head + 1]          # oldest frame -> receives the prediction
            self.model(ring, invariants=self.invariants, frame0=head, out=slot)
            r, a = ops.weighted_metrics_unnorm(slot, tg[i].view(1, 1, C, H, W), self.std, self.mean,
                                               self.weights, self.clim)
            rmse[i] = r.view(C)
            if acc is not None:
                acc[i] = a.view(C)
            if fields is not None:
                fields[i] = slot[0, 0]
            head = (head + 1) % T
        return rmse, acc, fields
