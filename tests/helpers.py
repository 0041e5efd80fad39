"""Shared test utilities: tolerances and comparisons against the CPU oracle."""
from __future__ import annotations

import numpy as np
import torch

# Parity bar for bf16 kernels against an fp32 reference on identical bf16-rounded inputs:
# the absolute bound of the specification (max-abs 2e-2, mean-abs 2e-3) and, next to it, a
# relative one (max-abs error <= 2e-2 * max|ref|, mean-abs error <= 2e-2 * mean|ref|), so
# that outputs of small magnitude are held to the same 2% as outputs of order one.
MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3
REL_TOL = 2e-2
# Floor of the relative bound (outputs that are all exactly zero).
_REL_FLOOR = 1e-6

# The same bar for fp16 kernels, four times tighter: fp16 keeps 11 significant bits to
# bf16's 8, so rounding P and the output costs about an eighth of the bf16 error.
F16_MAX_ABS_TOL = 5e-3
F16_MEAN_ABS_TOL = 5e-4
F16_REL_TOL = 5e-3


def bar(dtype: torch.dtype) -> dict[str, float]:
    """Keyword arguments of ``parity_failure`` / ``assert_close_bf16`` for a kernel dtype."""
    if dtype == torch.float16:
        return {"max_abs": F16_MAX_ABS_TOL, "mean_abs": F16_MEAN_ABS_TOL, "rel": F16_REL_TOL}
    return {"max_abs": MAX_ABS_TOL, "mean_abs": MEAN_ABS_TOL, "rel": REL_TOL}


def to_np(t: torch.Tensor) -> np.ndarray:
    """Float32 numpy copy of a (possibly bf16, possibly device) tensor."""
    return t.detach().float().cpu().numpy()


def parity_errors(actual: np.ndarray, expected: np.ndarray) -> dict[str, float]:
    """Absolute and relative error figures of ``actual`` against ``expected``."""
    err = np.abs(actual.astype(np.float64) - expected.astype(np.float64))
    ref = np.abs(expected.astype(np.float64))
    if err.size == 0:
        return {"max": 0.0, "mean": 0.0, "ref_max": 0.0, "ref_mean": 0.0}
    return {"max": float(err.max()), "mean": float(err.mean()),
            "ref_max": float(ref.max()), "ref_mean": float(ref.mean())}


def parity_failure(actual: np.ndarray, expected: np.ndarray, max_abs: float = MAX_ABS_TOL,
                   mean_abs: float = MEAN_ABS_TOL, rel: float | None = REL_TOL) -> str | None:
    """None if ``actual`` meets the bar against ``expected``, else a description."""
    if actual.shape != expected.shape:
        return f"shape {actual.shape} != {expected.shape}"
    if not np.isfinite(actual).all():
        return "non-finite values"
    e = parity_errors(actual, expected)
    bad = []
    if e["max"] > max_abs:
        bad.append(f"max-abs {e['max']:.3e} > {max_abs}")
    if e["mean"] > mean_abs:
        bad.append(f"mean-abs {e['mean']:.3e} > {mean_abs}")
    if rel is not None:
        if e["max"] > rel * e["ref_max"] + _REL_FLOOR:
            bad.append(f"max-abs {e['max']:.3e} > {rel} * max|ref| ({e['ref_max']:.3e})")
        if e["mean"] > rel * e["ref_mean"] + _REL_FLOOR:
            bad.append(f"mean-abs {e['mean']:.3e} > {rel} * mean|ref| ({e['ref_mean']:.3e})")
    return "; ".join(bad) or None


def assert_close_bf16(actual: torch.Tensor | np.ndarray, expected: np.ndarray, what: str,
                      max_abs: float = MAX_ABS_TOL, mean_abs: float = MEAN_ABS_TOL,
                      rel: float | None = REL_TOL) -> None:
    a = to_np(actual) if isinstance(actual, torch.Tensor) else np.asarray(actual, dtype=np.float32)
    fail = parity_failure(a, np.asarray(expected), max_abs, mean_abs, rel)
    assert fail is None, f"{what}: {fail}"


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def round_f16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest fp16 (ties to even), returned as float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def require_gpu() -> torch.device:
    assert torch.cuda.is_available(), "this test needs a ROCm GPU"
    return torch.device("cuda:0")


def write_bundle(root, gates, per_head, hidden_in_cfg=True, block_size=64, scalar_tau=0.5):
    """A bundle laid out as the reference exporter writes it (tasft/bundle/export.py:193-290):
    fp32 gate state dicts, kernel_config.json with the exporter's fields, manifest.json.

    ``gates`` maps layer index to an ``AttnGate``; ``per_head`` maps a layer index to its
    per-head thresholds (other layers get the scalar ``scalar_tau``)."""
    import hashlib
    import json

    from safetensors.torch import save_file

    (root / "gates").mkdir()
    (root / "model").mkdir()
    for i, g in gates.items():
        save_file({k: v.cpu().float() for k, v in g.state_dict().items()},
                  str(root / "gates" / f"layer_{i}_gate.safetensors"))
    (root / "model" / "model.safetensors").write_bytes(b"not read by the gate loader")
    layers = {}
    for i, g in gates.items():
        layers[str(i)] = {"layer_idx": i, "threshold_tau": scalar_tau, "target_sparsity": 0.7,
                          "achieved_sparsity_validation": 0.7, "gate_loss_validation": 0.0,
                          "block_size": block_size}
        if hidden_in_cfg:
            layers[str(i)]["gate_hidden_dim"] = g.gate_hidden_dim
        if i in per_head:
            layers[str(i)]["threshold_tau_per_head"] = [float(t) for t in per_head[i]]
    (root / "kernel_config.json").write_text(json.dumps(
        {"block_size": block_size, "global_threshold": scalar_tau, "per_layer_config": layers,
         "min_sparsity_for_speedup": 0.5}))
    files = sorted((root / "model").iterdir()) + sorted((root / "gates").iterdir()) + [root / "kernel_config.json"]
    sums = {str(f.relative_to(root)): hashlib.sha256(f.read_bytes()).hexdigest() for f in files}
    (root / "manifest.json").write_text(json.dumps({"model_name": "t", "num_layers": len(gates),
                                                    "checksums": sums}))
