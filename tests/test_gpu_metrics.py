"""GPU parity of the weighted RMSE / ACC kernel against the float64 numpy
oracle (utils/losses.py:243-266 restated), at the config-5 field size."""
import numpy as np
import pytest
import torch

from oracle import metrics_ref as mr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,T,C,H,W", [(1, 1, 70, 720, 1440), (2, 3, 4, 33, 50), (1, 1, 1, 1, 3)])
def test_rmse_acc_vs_oracle(device, B, T, C, H, W):
    import nsw
    g = np.random.default_rng(B * 100 + C)
    pred = g.standard_normal((B, T, C, H, W), dtype=np.float32)
    tgt = (pred + 0.3 * g.standard_normal((B, T, C, H, W), dtype=np.float32)).astype(np.float32)
    clim = g.standard_normal(C).astype(np.float32)
    w = mr.area_weights(mr.era5_latitudes(H))
    pt, tt = torch.from_numpy(pred).to(device), torch.from_numpy(tgt).to(device)
    wt = torch.from_numpy(w)[:, None]
    for ta in (True, False):
        rm = nsw.WeightedRMSE(wt, temporal_average=ta).to(device)(pt, tt).cpu().numpy()
        assert rm.dtype == np.float64
        np.testing.assert_allclose(rm, mr.weighted_rmse(pred, tgt, w, ta), rtol=1e-10, atol=0)
        ac = nsw.WeightedACC(wt, torch.from_numpy(clim), temporal_average=ta).to(device)(pt, tt).cpu().numpy()
        np.testing.assert_allclose(ac, mr.weighted_acc(pred, tgt, w, clim, ta), rtol=1e-10, atol=1e-12)


def test_rmse_full_weight_map_and_fp32_weights(device):
    """tests/test_metrics.py:59-64 of the reference uses a random [H, W] float32
    weight map; the product is then float32 in the reference, float64 here."""
    import nsw
    g = torch.Generator().manual_seed(5)
    B, T, C, H, W = 4, 2, 3, 72, 144
    pred = torch.randn(B, T, C, H, W, generator=g)
    tgt = torch.randn(B, T, C, H, W, generator=g)
    w = torch.rand(H, W, generator=g)
    got = nsw.WeightedRMSE(w).to(device)(pred.to(device), tgt.to(device)).cpu()
    want = torch.sqrt((w.double() * ((pred - tgt) ** 2).double()).sum((-1, -2)) / (H * W)).mean(0).mean(0)
    assert got.dtype == torch.float32   # float32 weights * float32 fields stay float32
    assert torch.allclose(got.double(), want, rtol=1e-6)


def test_rmse_special_cases(device):
    import nsw
    H, W = 720, 1440
    w = torch.from_numpy(mr.area_weights(mr.era5_latitudes(H)))
    p = torch.randn(1, 1, 2, H, W, device=device)
    m = nsw.WeightedRMSE(w[:, None]).to(device)
    assert torch.all(m(p, p) == 0)
    r = m(p + 0.5, p).cpu()
    assert torch.allclose(r, torch.full_like(r, 0.5), rtol=1e-6)
