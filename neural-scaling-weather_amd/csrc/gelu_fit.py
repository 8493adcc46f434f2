"""Coefficients of gelu_erf_bf16 (nsw_gemm_common.h): a least-squares fit
on Chebyshev nodes of log2(Phi(-a)), Phi the standard normal CDF, on
[0, 5.5] by a degree-5 polynomial in a, converted to monomial coefficients
and rounded to float32.  Run as a script it prints them (low order first)
and the worst error of the float32 Horner evaluation against float64 GELU
on a dense grid, in units of the bfloat16 half-ulp of the exact value.

GELU(v) = v Phi(v) = max(v, 0) - |v| Phi(-|v|), and Phi(-a) = exp2(P(a)).
"""
import numpy as np

DEGREE = 5
RANGE = 5.5


def fit(degree: int = DEGREE, a_max: float = RANGE) -> np.ndarray:
    from scipy.special import log_ndtr
    a = np.cos(np.linspace(0.0, np.pi, 8001)) * a_max / 2 + a_max / 2
    f = log_ndtr(-a) / np.log(2.0)
    c = np.polynomial.chebyshev.Chebyshev.fit(a, f, degree, domain=[0.0, a_max])
    return c.convert(kind=np.polynomial.Polynomial).coef.astype(np.float32)


def gelu_fast_f32(v: np.ndarray, coef: np.ndarray) -> np.ndarray:
    """float32 emulation of gelu_erf_bf16 (Horner from the top coefficient)."""
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v)
    p = np.full_like(a, coef[-1])
    with np.errstate(over="ignore", invalid="ignore"):   # huge |v|: P -> -inf, exp2 -> 0
        for c in coef[-2::-1]:
            p = (p * a + np.float32(c)).astype(np.float32)
        e = np.exp2(p).astype(np.float32)
    return (np.maximum(v, np.float32(0)) - a * e).astype(np.float32)


def bf16_half_ulp(x: np.ndarray) -> np.ndarray:
    e = np.floor(np.log2(np.maximum(np.abs(x), 1e-300)))
    return 2.0 ** (e - 8)


if __name__ == "__main__":
    from scipy.special import ndtr
    coef = fit()
    print(f"coefficients (a^0 .. a^{DEGREE}):", ", ".join(f"{float(c):.9e}f" for c in coef))
    v = np.linspace(-12, 12, 2_400_001).astype(np.float32)
    exact = v.astype(np.float64) * ndtr(v.astype(np.float64))
    got = gelu_fast_f32(v, coef).astype(np.float64)
    big = np.abs(exact) >= 2.0 ** -24
    print("max |err| / bf16 half-ulp:", (np.abs(got - exact)[big] / bf16_half_ulp(exact[big])).max())
