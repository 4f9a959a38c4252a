"""Shared fixtures: seeded models and inputs of the benchmark configurations, oracle adapters.

Seeds follow the measurement plan: weights torch.manual_seed(42) with PyTorch's default init,
x = randn(B, T, I) from Generator.manual_seed(1), ragged lengths randint(200, 1001) from
Generator.manual_seed(2) sorted descending, h0 = c0 = 0.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from persistent_lstm_hip_amd.model import StandardLSTMRegressor  # noqa: E402

# The accepted error of the fp16 GPU forward against the fp32 CPU oracle (output and per-step h/c).
MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


def make_regressor(I: int, H: int, L: int, O: int, seed: int = 42) -> StandardLSTMRegressor:
    torch.manual_seed(seed)
    return StandardLSTMRegressor(I, H, O, L).eval()


def make_x(B: int, T: int, I: int, seed: int = 1) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, T, I, generator=g)


def make_lengths(B: int, T: int, lo: int, seed: int = 2) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, T + 1, (B,), generator=g)
    return torch.sort(lens, descending=True).values


def oracle_layers(lstm: torch.nn.LSTM, half: bool = False):
    """(w_ih, w_hh, b_ih, b_hh) float32 numpy arrays per layer; half=True rounds them to fp16 first."""
    out = []
    for l in range(lstm.num_layers):
        ts = [getattr(lstm, f"{n}_l{l}").detach().float().cpu() for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")]
        if half:
            ts = [t.half().float() for t in ts]
        out.append(tuple(t.numpy() for t in ts))
    return out


def linear_params(linear: torch.nn.Linear, half: bool = False):
    w, b = linear.weight.detach().float().cpu(), linear.bias.detach().float().cpu()
    if half:
        w, b = w.half().float(), b.half().float()
    return w.numpy(), b.numpy()


def assert_close(got, want, max_abs=MAX_ABS_TOL, mean_abs=MEAN_ABS_TOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    d = np.abs(got - want)
    assert d.max() <= max_abs and d.mean() <= mean_abs, (
        f"{what}: max_abs={d.max():.3e} (tol {max_abs}) mean_abs={d.mean():.3e} (tol {mean_abs})")
    return float(d.max()), float(d.mean())


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.fail("a HIP GPU is required for tests marked gpu")
    from persistent_lstm_hip_amd.extension import require_extension

    return require_extension()
