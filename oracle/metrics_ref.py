"""Latitude-weighted RMSE / ACC and area weights (test oracle only).

* :func:`area_weights` restates ``build_spherical_area_weights``
  (utils/misc_utils.py:41-52): cos(lat) / mean(cos(lat)) in float64, used as
  ``[nlat, 1]`` (utils/dataloaders/era5hdf5.py:159) on the ERA5 latitudes with
  the south pole dropped (era5hdf5.py:208).
* :func:`weighted_rmse` restates ``WeightedRMSE.forward`` (utils/losses.py:243-266)
  in the dtypes the reference ends up with: the difference and its square are
  fp32 (pred and target are fp32), the float64 weights promote the product and
  the spatial sum to float64, then sqrt(sum / (H*W)) and means over the batch
  (and time when ``temporal_average``).
* :func:`weighted_acc` is the textbook latitude-weighted anomaly correlation
  (not present in the reference): with a = x - clim[c],
  acc = sum(w a_f a_o) / sqrt(sum(w a_f^2) * sum(w a_o^2)).

Pinning (tests/test_oracle_metrics.py): brute-force double loops on tiny
fields; p == t -> 0; a constant offset d -> |d| (weights have mean 1);
f == o -> acc 1; f - clim == -(o - clim) -> acc -1.
"""
from __future__ import annotations

import numpy as np


def era5_latitudes(nlat: int = 720) -> np.ndarray:
    """ERA5 0.25 deg latitudes 90 .. -90 (721 rows) with the south pole dropped."""
    return np.linspace(90.0, -90.0, nlat + 1)[:-1]


def area_weights(latitudes: np.ndarray) -> np.ndarray:
    c = np.cos(np.deg2rad(latitudes))
    return c / c.mean()


def weighted_sums(pred: np.ndarray, target: np.ndarray, w_lat: np.ndarray,
                  clim: np.ndarray | None = None, field_dtype=np.float32) -> np.ndarray:
    """Per (b, t, c) plane: [sum w*(p-t)^2, sum w*af*ao, sum w*af^2, sum w*ao^2]
    (float64).  pred/target [B,T,C,H,W] holding values of ``field_dtype``
    (float32 fields, or float64 ones when float64 statistics promoted them),
    in which the difference and its square are formed; w_lat [H]; clim [C]
    or None."""
    fd = np.dtype(field_dtype)
    p = pred.astype(fd)
    t = target.astype(fd)
    d = (p - t).astype(fd)
    se = (d * d).astype(fd).astype(np.float64)
    w = w_lat.astype(np.float64)[:, None]
    out = np.zeros(pred.shape[:3] + (4,), dtype=np.float64)
    out[..., 0] = (se * w).sum(axis=(-1, -2))
    if clim is not None:
        cl = clim.astype(fd)[None, None, :, None, None]
        af = (p - cl).astype(fd).astype(np.float64)
        ao = (t - cl).astype(fd).astype(np.float64)
        out[..., 1] = (w * af * ao).sum(axis=(-1, -2))
        out[..., 2] = (w * af * af).sum(axis=(-1, -2))
        out[..., 3] = (w * ao * ao).sum(axis=(-1, -2))
    return out


def weighted_rmse(pred, target, w_lat, temporal_average: bool = True, field_dtype=np.float32) -> np.ndarray:
    H, W = pred.shape[-2:]
    s = weighted_sums(pred, target, w_lat, field_dtype=field_dtype)[..., 0]
    rmse = np.sqrt(s / float(H * W))        # [B, T, C]
    if temporal_average:
        while rmse.ndim > 1:
            rmse = rmse.mean(axis=0)
        return rmse
    return rmse.mean(axis=0)


def weighted_acc(pred, target, w_lat, clim, temporal_average: bool = True, field_dtype=np.float32) -> np.ndarray:
    s = weighted_sums(pred, target, w_lat, clim, field_dtype=field_dtype)
    acc = s[..., 1] / np.sqrt(s[..., 2] * s[..., 3])
    if temporal_average:
        while acc.ndim > 1:
            acc = acc.mean(axis=0)
        return acc
    return acc.mean(axis=0)


def weighted_sums_bruteforce(pred, target, w_lat, clim=None):
    """Scalar-loop version of :func:`weighted_sums` (tiny fields only)."""
    B, T, C, H, W = pred.shape
    out = np.zeros((B, T, C, 4), dtype=np.float64)
    for b in range(B):
        for t in range(T):
            for c in range(C):
                acc = [0.0, 0.0, 0.0, 0.0]
                for h in range(H):
                    wh = float(w_lat[h])
                    for x in range(W):
                        pv = np.float32(pred[b, t, c, h, x])
                        tv = np.float32(target[b, t, c, h, x])
                        d = np.float32(pv - tv)
                        acc[0] += wh * float(np.float32(d * d))
                        if clim is not None:
                            af = float(np.float32(pv - np.float32(clim[c])))
                            ao = float(np.float32(tv - np.float32(clim[c])))
                            acc[1] += wh * af * ao
                            acc[2] += wh * af * af
                            acc[3] += wh * ao * ao
                out[b, t, c] = acc
    return out
