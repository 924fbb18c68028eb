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


def or_rule_violations(got, want, atol=0.002, rtol=0.02):
    """Count elements failing |d| <= atol OR |d| <= rtol*|ref| (non-finite fails)."""
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    err = (got - want).abs()
    ok = torch.isfinite(got) & torch.isfinite(want) & ((err <= atol) | (err <= rtol * want.abs()))
    return int((~ok).sum()), float(err.max()) if err.numel() else 0.0
