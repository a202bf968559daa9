"""Shared test helpers.

GPU tests are marked ``gpu`` and compare the native HIP path with the CPU
oracle in ``oracle/``.  Tolerance for bf16 outputs and gradients against the
fp32 oracle (stated once, used everywhere):
    max |a - r| <= 2e-2 * max(1, max |r|)   and   ||a - r||_2 / ||r||_2 <= 1e-2
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MAX_ABS = 2e-2
REL_L2 = 1e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X) and the built liblighthouse_hip.so")


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__ as G
    return G.load_package()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def assert_close(a, r, name, max_abs=MAX_ABS, rel_l2=REL_L2):
    """bf16-vs-fp32 tolerance check; returns (max error, relative L2)."""
    import torch
    a = a.detach().float().cpu()
    r = r.detach().float().cpu()
    assert a.shape == r.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(r.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    err = (a - r).abs().max().item() if a.numel() else 0.0
    den = r.norm().item()
    rel = ((a - r).norm().item() / den) if den > 0 else (a.norm().item())
    bound = max_abs * max(1.0, r.abs().max().item() if r.numel() else 1.0)
    assert err <= bound and rel <= rel_l2, f"{name}: max-abs {err:.3e} (bound {bound:.3e}), rel-L2 {rel:.3e}"
    return err, rel
