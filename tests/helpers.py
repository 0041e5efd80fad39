"""Shared test utilities: tolerances and comparisons against the CPU oracle."""
from __future__ import annotations

import numpy as np
import torch

# Parity bar for bf16 kernels against an fp32 reference on identical bf16-rounded inputs.
MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3


def to_np(t: torch.Tensor) -> np.ndarray:
    """Float32 numpy copy of a (possibly bf16, possibly device) tensor."""
    return t.detach().float().cpu().numpy()


def assert_close_bf16(actual: torch.Tensor | np.ndarray, expected: np.ndarray, what: str,
                      max_abs: float = MAX_ABS_TOL, mean_abs: float = MEAN_ABS_TOL) -> None:
    a = to_np(actual) if isinstance(actual, torch.Tensor) else np.asarray(actual, dtype=np.float32)
    assert a.shape == expected.shape, f"{what}: shape {a.shape} != {expected.shape}"
    assert np.isfinite(a).all(), f"{what}: non-finite values in kernel output"
    err = np.abs(a.astype(np.float64) - expected.astype(np.float64))
    mx, mn = float(err.max()) if err.size else 0.0, float(err.mean()) if err.size else 0.0
    assert mx <= max_abs and mn <= mean_abs, (
        f"{what}: max-abs {mx:.3e} (tol {max_abs}), mean-abs {mn:.3e} (tol {mean_abs})")


def require_gpu() -> torch.device:
    assert torch.cuda.is_available(), "this test needs a ROCm GPU"
    return torch.device("cuda:0")
