"""Pins the oracle's RMSE / ACC / area weights: brute force and closed forms."""
import numpy as np
import pytest

from oracle import metrics_ref as mr


def test_area_weights_closed_form():
    lat = mr.era5_latitudes(720)
    assert lat.shape == (720,) and lat[0] == 90.0 and abs(lat[-1] + 89.75) < 1e-12
    w = mr.area_weights(lat)
    assert abs(w.mean() - 1.0) < 1e-14
    assert w[0] < 1e-15 + abs(np.cos(np.pi / 2)) / np.cos(np.deg2rad(lat)).mean()
    # symmetric about the equator except for the dropped south pole
    assert np.allclose(w[1:360], w[719:360:-1], rtol=1e-12)


def test_sums_vs_bruteforce():
    rng = np.random.default_rng(0)
    B, T, C, H, W = 2, 1, 3, 4, 6
    p = rng.standard_normal((B, T, C, H, W)).astype(np.float32)
    t = rng.standard_normal((B, T, C, H, W)).astype(np.float32)
    w = mr.area_weights(mr.era5_latitudes(H))
    clim = rng.standard_normal(C).astype(np.float32)
    a = mr.weighted_sums(p, t, w, clim)
    b = mr.weighted_sums_bruteforce(p, t, w, clim)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_rmse_special_cases():
    rng = np.random.default_rng(1)
    B, T, C, H, W = 1, 2, 3, 8, 16
    p = rng.standard_normal((B, T, C, H, W)).astype(np.float32)
    w = mr.area_weights(mr.era5_latitudes(H))
    assert np.all(mr.weighted_rmse(p, p, w) == 0)
    d = np.float32(0.5)
    r = mr.weighted_rmse(p + d, p, w, temporal_average=False)
    assert r.shape == (T, C)
    assert np.allclose(r, 0.5, rtol=1e-6)


def test_acc_special_cases():
    rng = np.random.default_rng(2)
    B, T, C, H, W = 1, 1, 2, 8, 16
    clim = rng.standard_normal(C).astype(np.float32)
    f = rng.standard_normal((B, T, C, H, W)).astype(np.float32)
    w = mr.area_weights(mr.era5_latitudes(H))
    assert np.allclose(mr.weighted_acc(f, f, w, clim), 1.0, atol=1e-12)
    o = (2 * clim[None, None, :, None, None] - f).astype(np.float32)
    assert np.allclose(mr.weighted_acc(f, o, w, clim), -1.0, atol=1e-6)


def test_float64_fields_keep_float64_differences():
    """With float64 fields (float64 statistics promote the unnormalised
    fields) the squared differences are formed in float64: a float64 offset
    that float32 cannot hold is recovered exactly, and the sums equal a
    float64 loop."""
    rng = np.random.default_rng(3)
    B, T, C, H, W = 1, 1, 2, 4, 6
    p = rng.standard_normal((B, T, C, H, W)) * 10
    d = 1e-9
    w = mr.area_weights(mr.era5_latitudes(H))
    r64 = mr.weighted_rmse(p + d, p, w, field_dtype=np.float64)
    assert np.allclose(r64, d, rtol=1e-4, atol=0)
    assert not np.allclose(mr.weighted_rmse(p + d, p, w), d, rtol=1e-4, atol=0)     # float32 fields lose it
    t = rng.standard_normal((B, T, C, H, W))
    s = mr.weighted_sums(p, t, w, field_dtype=np.float64)[..., 0]
    brute = np.zeros((B, T, C))
    for c in range(C):
        brute[0, 0, c] = sum(w[h] * (p[0, 0, c, h, x] - t[0, 0, c, h, x]) ** 2 for h in range(H) for x in range(W))
    assert np.allclose(s, brute, rtol=1e-13)
