"""Fit the polynomial of the GELU epilogue (gelu_erf in tk_common.hpp).

    python fit_gelu.py        # prints the coefficients and the error of the fp32 formula

GELU(x) = x*Phi(x) = max(x, 0) - a*Phi(-a) with a = |x| (x - x*Phi(-x) for x >= 0, x*Phi(x)
for x < 0), so only the tail r(a) = a*Phi(-a) >= 0 has to be approximated.  log2 Phi(-a) is
smooth and concave on [0, inf) (-1 at 0, ~ -a^2/(2 ln 2) for large a), so r(a) = a * 2^P(a)
with a short polynomial P.  P(0) = -1 is fixed (GELU(x) ~ x/2 to the last bit near 0) and
c1..c5 minimise max |a*2^P(a) - r(a)| over a dense grid of [0, 10]: a linear program in the
coefficients after weighting the error in P by r(a)*ln 2 (its first-order effect on r).  The
leading coefficient comes out negative, so P keeps falling beyond the fitted range and 2^P
underflows to 0 instead of growing.  The device evaluates P by Horner in fp32 (5 FMAs), one
v_exp_f32 and one final FMA: max(x, 0) - a*2^P(a).
"""
from __future__ import annotations

import numpy as np
from scipy.optimize import linprog
from scipy.special import log_ndtr

DEGREE, A_MAX, POINTS = 5, 10.0, 20000


def fit() -> np.ndarray:
    a = np.linspace(0.0, A_MAX, POINTS)
    target = log_ndtr(-a) / np.log(2.0)                  # log2 Phi(-a)
    w = np.log(2.0) * a * np.exp(log_ndtr(-a))           # d r / d P
    basis = np.vander(a, DEGREE + 1, increasing=True)[:, 1:] * w[:, None]
    rhs = (target + 1.0) * w                             # c0 = -1 moved to the right
    n = DEGREE
    cost = np.zeros(n + 1)
    cost[-1] = 1.0                                       # minimise the bound e
    a_ub = np.vstack([np.hstack([basis, -np.ones((POINTS, 1))]),
                      np.hstack([-basis, -np.ones((POINTS, 1))])])
    b_ub = np.concatenate([rhs, -rhs])
    res = linprog(cost, A_ub=a_ub, b_ub=b_ub, bounds=[(None, None)] * n + [(0, None)], method="highs")
    if not res.success:
        raise RuntimeError(res.message)
    return np.concatenate([[-1.0], res.x[:n]]).astype(np.float32)


def gelu_fp32(x: np.ndarray, coef) -> np.ndarray:
    """The device formula in fp32 (each FMA rounded once, as v_fma_f32)."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    c = [np.float64(np.float32(v)) for v in coef]
    p = np.float64(c[-1])
    with np.errstate(over="ignore"):  # P -> -inf in fp32 for huge |x|, as on the device
        for k in range(len(c) - 2, -1, -1):
            p = (p * a + c[k]).astype(np.float32).astype(np.float64)
        e = np.exp2(p).astype(np.float32).astype(np.float64)
        return (np.maximum(x.astype(np.float64), 0.0) - a * e).astype(np.float32)


def gelu_exact(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    return np.maximum(x, 0.0) - a * np.exp(log_ndtr(-a))


if __name__ == "__main__":
    coef = fit()
    print("coefficients c0..c5:", ", ".join(f"{float(v):.9e}" for v in coef))
    x = np.linspace(-12.0, 12.0, 2_400_001, dtype=np.float32)
    err = np.abs(gelu_fp32(x, coef).astype(np.float64) - gelu_exact(x))
    print(f"max |GELU error| on [-12, 12]: {err.max():.3e}")
