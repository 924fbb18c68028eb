"""Shared test setup: import paths, the ``gpu`` marker, seeded helpers."""

from __future__ import annotations

import os
import pathlib
import sys

import pytest
import torch

REPO = pathlib.Path(__file__).resolve().parents[1]
PKG_PARENT = REPO / "transformer-kernel_amd"
for p in (str(REPO), str(PKG_PARENT)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN_DIR = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtkmi.so")
    config.addinivalue_line("markers", "slow: long-running parity case (full-size configs)")


# Worst parity margin per benchmark config over every checked trial:
# config -> {"max_abs", "budget_frac", "trials"}.  budget_frac is the largest
# |d| / max(atol, rtol * |ref|) over the elements (1.0 = on the harness's
# limit, src/torch_transformer_benchmark.py:309-316); the terminal summary
# prints it so the GPU run's log carries the margins, not only a pass count.
PARITY_MARGINS = {}


def budget_fraction(ref, got, atol=0.002, rtol=0.02):
    """Largest share of the per-element tolerance used (inf if anything is non-finite)."""
    ref = ref.detach().float().cpu()
    got = got.detach().float().cpu()
    if not (torch.isfinite(ref).all() and torch.isfinite(got).all()):
        return float("inf")
    lim = torch.clamp(ref.abs() * rtol, min=atol)
    return float(((got - ref).abs() / lim).max()) if ref.numel() else 0.0


def record_parity(config: str, ref, got, max_abs: float) -> None:
    frac = budget_fraction(ref, got)
    cur = PARITY_MARGINS.setdefault(config, {"max_abs": 0.0, "budget_frac": 0.0, "trials": 0})
    cur["max_abs"] = max(cur["max_abs"], float(max_abs))
    cur["budget_frac"] = max(cur["budget_frac"], frac)
    cur["trials"] += 1


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    if not PARITY_MARGINS:
        return
    tr = terminalreporter
    tr.write_line("parity margins (worst over the checked trials; budget |d| <= 0.002 or <= 0.02*|ref|):")
    for name in sorted(PARITY_MARGINS):
        m = PARITY_MARGINS[name]
        tr.write_line(f"  {name}: max|d| {m['max_abs']:.3e}, {100.0 * m['budget_frac']:.1f}% of the "
                      f"element budget, {m['trials']} trials")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True, scope="session")
def _cpu_threads():
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    torch.set_float32_matmul_precision("highest")
    yield


def seeded(*shape, dtype=torch.float32, seed=0, scale=1.0, device="cpu"):
    """randn from a seeded CPU generator, then moved (src/test_triton_kernels.py:52-55 recipe)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    t = torch.randn(*shape, generator=g, dtype=torch.float32) * scale
    return t.to(device=device, dtype=dtype)


def fp16_excess(got, want, atol):
    """Largest amount by which |got - want| exceeds max(atol, one fp16 ulp of want).

    An fp16 output may differ from the reference's fp16 cast by one ulp where a
    different fp32 accumulation order lands on the other side of a rounding
    boundary (the reference's own note, src/test_kernels.py:61-63); at |x| in
    [2, 4) one ulp is 0.00195, above a flat 1e-3.
    """
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    mag = want.abs().clamp_min(2.0 ** -14)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 10)
    return float(((got - want).abs() - torch.maximum(ulp, torch.full_like(ulp, atol))).max())


def or_rule_violations(got, want, atol=0.002, rtol=0.02):
    """Count elements failing |d| <= atol OR |d| <= rtol*|ref| (non-finite fails)."""
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    err = (got - want).abs()
    ok = torch.isfinite(got) & torch.isfinite(want) & ((err <= atol) | (err <= rtol * want.abs()))
    return int((~ok).sum()), float(err.max()) if err.numel() else 0.0
