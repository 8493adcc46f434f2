"""The allocation-free metrics entry point (nsw_weighted_metrics_unnorm_noalloc,
library-owned per-GPU scratch) against the workspace entry point it varies
(nsw_weighted_metrics_unnorm), called through the C ABI: two calls in a row,
the second on a smaller input, bit-identical results (same kernels, same
fixed reduction order); inputs beyond the scratch are refused before any
launch."""
import ctypes

import pytest
import torch

from oracle import metrics_ref

pytestmark = pytest.mark.gpu


def fields(P, H, W, seed, pred_dtype):
    g = torch.Generator().manual_seed(seed)
    pred = torch.randn(P, H, W, generator=g).to(pred_dtype)
    tgt = torch.randn(P, H, W, generator=g)
    return pred, tgt


def call_both(device, C, S, H, W, pred_dtype, seed):
    """S time steps x C channels = P planes of H x W through both entry points."""
    from nsw import _lib
    L = _lib.lib()
    P = S * C
    pred, tgt = fields(P, H, W, seed, pred_dtype)
    g = torch.Generator().manual_seed(seed + 1)
    std = torch.rand(C, generator=g) + 0.5
    mean = torch.randn(C, generator=g) * 10
    clim = torch.randn(C, generator=g) * 10
    w = torch.from_numpy(metrics_ref.area_weights(metrics_ref.era5_latitudes(H)))
    d = {k: v.to(device).contiguous() for k, v in dict(pred=pred, tgt=tgt, std=std, mean=mean, clim=clim,
                                                       w=w).items()}
    dt = _lib.NSW_DTYPE_BF16 if pred_dtype == torch.bfloat16 else _lib.NSW_DTYPE_F32
    stream = torch.cuda.current_stream(device).cuda_stream
    out = {}
    for name in ("ws", "noalloc"):
        rmse = torch.full((P,), -1.0, dtype=torch.float64, device=device)
        acc = torch.full((P,), -1.0, dtype=torch.float64, device=device)
        if name == "ws":
            nbytes = L.nsw_weighted_metrics_workspace_size(P, H, W)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            rc = L.nsw_weighted_metrics_unnorm(d["pred"].data_ptr(), dt, d["tgt"].data_ptr(), d["std"].data_ptr(),
                                               d["mean"].data_ptr(), d["w"].data_ptr(), 1, d["clim"].data_ptr(),
                                               P, H, W, C, rmse.data_ptr(), acc.data_ptr(), ws.data_ptr(),
                                               nbytes, stream)
        else:
            rc = L.nsw_weighted_metrics_unnorm_noalloc(d["pred"].data_ptr(), dt, d["tgt"].data_ptr(),
                                                       d["std"].data_ptr(), d["mean"].data_ptr(), d["w"].data_ptr(),
                                                       1, d["clim"].data_ptr(), P, H, W, C, rmse.data_ptr(),
                                                       acc.data_ptr(), stream)
        assert rc == 0, L.nsw_last_error()
        torch.cuda.synchronize()
        out[name] = (rmse.cpu(), acc.cpu())
    return out


@pytest.mark.parametrize("pred_dtype", [torch.float32, torch.bfloat16])
def test_noalloc_matches_workspace_entry_point(device, pred_dtype):
    # first call: one config-5 step (70 channels on the 720 x 1440 grid)
    big = call_both(device, 70, 1, 720, 1440, pred_dtype, seed=3)
    # second call, smaller: 2 steps x 5 channels on a 90 x 180 grid; the
    # scratch still holds the first call's partial sums
    small = call_both(device, 5, 2, 90, 180, pred_dtype, seed=4)
    for out in (big, small):
        assert torch.equal(out["noalloc"][0], out["ws"][0])
        assert torch.equal(out["noalloc"][1], out["ws"][1])
        assert torch.all(out["noalloc"][0] > 0)


def test_noalloc_refuses_inputs_beyond_the_scratch(device):
    from nsw import _lib
    L = _lib.lib()
    P, H, W = 40000, 720, 1440
    assert L.nsw_weighted_metrics_workspace_size(P, H, W) > _lib.NSW_METRICS_SCRATCH_BYTES
    stream = torch.cuda.current_stream(device).cuda_stream
    # refused on the host before any pointer is touched
    rc = L.nsw_weighted_metrics_unnorm_noalloc(ctypes.c_void_p(16), _lib.NSW_DTYPE_F32, ctypes.c_void_p(16),
                                               ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 1,
                                               None, P, H, W, 70, ctypes.c_void_p(16), None, stream)
    assert rc == _lib.NSW_ERR_INVALID
    assert b"scratch" in L.nsw_last_error()
