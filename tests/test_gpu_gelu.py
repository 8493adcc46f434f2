"""GPU check of the GELU epilogue of the bfloat16 GEMM (gelu_erf_bf16 in the
fc1 epilogue) on every finite bfloat16 value in [-12, 12]: y = GELU(x . I^T)
through nsw_linear, whose fp32 accumulation reproduces x exactly.  Each
output is within 1.15 bfloat16 half-ulps of the float64 exact-erf GELU
(v Phi(v), models/mlp.py:55): the rounding of a value within 0.145 half-ulps
of exact (the fit's worst case, for negative v); outputs whose exact value
is below 2^-24 stay below 2^-22.  The fp32 epilogue (A&S 7.1.26) is checked against
F.gelu in test_gpu_kernels.py."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_bf16_gelu_epilogue_dense_grid(device):
    special = pytest.importorskip("scipy.special")
    from nsw import _lib, ops
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    vals = bits.view(torch.bfloat16).float()
    vals = vals[torch.isfinite(vals) & (vals.abs() <= 12)]
    K = 64
    n = vals.numel()
    M = -(-n // K)
    x = torch.zeros(M * K)
    x[:n] = vals
    x = x.view(M, K).to(device, torch.bfloat16)
    w = torch.eye(K, device=device, dtype=torch.bfloat16)
    b = torch.zeros(K, device=device, dtype=torch.bfloat16)
    y = ops.linear(x, w, b, epilogue=_lib.NSW_EPI_BIAS_GELU)
    torch.cuda.synchronize()
    got = y.float().cpu().reshape(-1)[:n].double().numpy()
    v = vals.double().numpy()
    exact = v * special.ndtr(v)
    big = np.abs(exact) >= 2.0 ** -24
    e = np.floor(np.log2(np.abs(exact[big])))
    half_ulp = 2.0 ** (e - 8)
    ratio = np.abs(got[big] - exact[big]) / half_ulp
    assert ratio.max() <= 1.15, (v[big][ratio.argmax()], got[big][ratio.argmax()], exact[big][ratio.argmax()])
    assert np.abs(got[~big]).max() < 2.0 ** -22
