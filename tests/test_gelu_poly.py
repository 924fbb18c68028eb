"""The GELU epilogue's formula (gelu_erf in transformer-kernel_amd/csrc/tk_common.hpp), on the CPU.

The device computes GELU(x) = max(x, 0) - |x| * 2^P(|x|) with a degree-5 polynomial P that
fit_gelu.py (beside the kernel sources) fits.  These tests read the coefficients out of the
kernel source, evaluate the same fp32 operations in numpy and compare with the exact-erf GELU
in float64 (x * Phi(x) through scipy's log_ndtr), so a wrong coefficient, a dropped term or a
sign error in the source fails here before any GPU run.  The GPU test
test_gelu_epilogue_dense_range checks the compiled epilogue against the same exact GELU.
"""
from __future__ import annotations

import importlib.util
import math
import pathlib
import re

import numpy as np
import pytest

CSRC = pathlib.Path(__file__).resolve().parents[1] / "transformer-kernel_amd" / "csrc"
spec = importlib.util.spec_from_file_location("fit_gelu", CSRC / "fit_gelu.py")
fg = importlib.util.module_from_spec(spec)
spec.loader.exec_module(fg)


def source_coefficients() -> list[float]:
    """c0..c5 of P as the kernel source writes them (Horner from c5 down)."""
    src = (CSRC / "tk_common.hpp").read_text()
    body = src[src.index("float gelu_erf(float x)"):]
    body = body[:body.index("\n}\n")]
    lits = [float(v) for v in re.findall(r"([-+]?\d\.\d+e[-+]\d+|-1\.0)f", body)]
    c5, c4, c3, c2, c1, c0 = lits
    return [c0, c1, c2, c3, c4, c5]


def test_source_coefficients_are_the_fit():
    got = np.array(source_coefficients(), dtype=np.float32)
    want = fg.fit()
    assert got[0] == -1.0
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=0)


def test_formula_matches_exact_gelu():
    x = np.linspace(-12.0, 12.0, 1_200_001, dtype=np.float32)
    got = fg.gelu_fp32(x, source_coefficients()).astype(np.float64)
    want = fg.gelu_exact(x)
    assert np.abs(got - want).max() <= 7.2e-7
    # near 0, GELU(x) ~ x/2: relative error too
    small = x[(np.abs(x) > 0) & (np.abs(x) < 1e-2)]
    rel = np.abs(fg.gelu_fp32(small, source_coefficients()) / fg.gelu_exact(small) - 1)
    assert rel.max() <= 1e-6
    # spot values from math.erf
    for v in (-3.0, -1.0, -0.5, 0.25, 1.0, 2.5):
        exact = 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0)))
        assert abs(float(fg.gelu_fp32(np.float32(v), source_coefficients())) - exact) <= 7.2e-7


def test_formula_tails_are_finite():
    big = np.geomspace(12.0, 3.0e38, 4000).astype(np.float32)
    pos = fg.gelu_fp32(big, source_coefficients())
    neg = fg.gelu_fp32(-big, source_coefficients())
    assert np.all(np.isfinite(pos)) and np.all(np.isfinite(neg))
    assert np.all(pos == big)               # GELU(x) = x to fp32 precision
    assert np.abs(neg).max() <= 1e-30       # and 0 for large negative x


@pytest.mark.parametrize("plant", ["c1_sign", "c5_dropped", "c0_half"])
def test_checks_catch_planted_mistakes(plant):
    c = source_coefficients()
    if plant == "c1_sign":
        c[1] = -c[1]
    elif plant == "c5_dropped":
        c[5] = 0.0
    else:
        c[0] = -0.5
    x = np.linspace(-12.0, 12.0, 200_001, dtype=np.float32)
    err = np.abs(fg.gelu_fp32(x, c).astype(np.float64) - fg.gelu_exact(x)).max()
    assert not err <= 7.2e-7
