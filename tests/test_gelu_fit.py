"""The bfloat16-output GELU of the fc1 epilogue (gelu_erf_bf16 in
nsw_gemm_common.h): its coefficients are those csrc/gelu_fit.py derives, and
its float32 evaluation stays within 0.15 of a bfloat16 half-ulp of the
float64 exact-erf GELU (v Phi(v), models/mlp.py:55's nn.GELU()) on a dense
grid; past the fitted range the exponent keeps falling, so large |v| give v
(v > 0) or values below 2^-22 in magnitude (v < 0)."""
import importlib.util
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "neural-scaling-weather_amd", "csrc")


def _fit_module():
    spec = importlib.util.spec_from_file_location("gelu_fit", os.path.join(CSRC, "gelu_fit.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def header_coefficients():
    src = open(os.path.join(CSRC, "nsw_gemm_common.h")).read()
    body = src[src.index("float gelu_erf_bf16(float v)"):]
    body = body[:body.index("\n}\n")]
    nums = [float(x) for x in re.findall(r"([-+]?\d\.\d+e[-+]\d+)f", body)]
    # fmaf(c5, a, c4), then c3 .. c0 (Horner from the top)
    return np.array(nums[::-1], dtype=np.float32)


def test_header_matches_fit():
    pytest.importorskip("scipy")
    fit = _fit_module().fit()
    coef = header_coefficients()
    assert coef.shape == fit.shape == (6,)
    np.testing.assert_allclose(coef, fit, rtol=1e-6)


def test_error_below_bf16_half_ulp():
    special = pytest.importorskip("scipy.special")
    mod = _fit_module()
    coef = header_coefficients()
    v = np.linspace(-12, 12, 2_400_001).astype(np.float32)
    v = np.concatenate([v, np.float32([0.0, -0.0, 1e-30, -1e-30, 5.5, -5.5])])
    exact = v.astype(np.float64) * special.ndtr(v.astype(np.float64))
    got = mod.gelu_fast_f32(v, coef).astype(np.float64)
    big = np.abs(exact) >= 2.0 ** -24
    ratio = np.abs(got - exact)[big] / mod.bf16_half_ulp(exact[big])
    assert ratio.max() < 0.15
    assert np.abs(got[~big]).max() < 2.0 ** -22


def test_tail_beyond_fit_range():
    coef = header_coefficients().astype(np.float64)
    a = np.linspace(5.5, 1000.0, 200_001)
    p = np.polyval(coef[::-1], a)
    assert np.all(np.diff(p) < 0) and p[0] < -25
    mod = _fit_module()
    big = np.float32([20.0, 100.0, 1e4, 1e30])
    np.testing.assert_array_equal(mod.gelu_fast_f32(big, header_coefficients()), big)
    assert np.all(np.abs(mod.gelu_fast_f32(-big, header_coefficients())) < 2.0 ** -22)
