"""The gate side of a TASFT bundle: per-layer AttnGates and thresholds.

A bundle (written by the reference exporter, ``tasft/bundle/export.py:193-290``) holds
``gates/layer_{i}_gate.safetensors`` (fp32 state dicts), ``kernel_config.json`` and
``manifest.json`` (SHA-256 of every file). The reference loader
(``tasft/inference/tasft_model.py:521-580``) builds every gate with the default hidden width
(``AttnGate(num_heads, head_dim, block_size)``, no ``gate_hidden_dim``), so a gate trained
with another width fails ``load_state_dict``, and it gives every layer one scalar tau.

``load_bundle_gates`` builds each gate with the width its state dict was trained with
(checked against ``LayerKernelConfig.gate_hidden_dim`` when the config records it), the
layer's block size, and the layer's per-head thresholds when ``threshold_tau_per_head`` is
present (else the scalar tau). The merged base model in ``model/`` is not read (loading an
HF model is outside this path); its checksum is verified only when ``verify`` includes it.
"""
from __future__ import annotations

import hashlib
import json
import re
from dataclasses import dataclass
from pathlib import Path

import torch

from tasft_amd.exceptions import BundleError, ChecksumError
from tasft_amd.kernels.kernel_config import KernelConfig
from tasft_amd.modules.attn_gate import AttnGate

_GATE_FILE = re.compile(r"^layer_(\d+)_gate\.safetensors$")


@dataclass(frozen=True)
class BundleGates:
    """Gates of a bundle, by layer index, with their thresholds and the kernel config.

    ``thresholds[i]`` is a float, or a ``[num_heads]`` fp32 tensor when the layer records
    per-head thresholds (``AttnGate.forward(threshold=...)`` takes either)."""

    gates: dict[int, AttnGate]
    thresholds: dict[int, float | torch.Tensor]
    block_sizes: dict[int, int]
    kernel_config: KernelConfig


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(65536), b""):
            h.update(chunk)
    return h.hexdigest()


def _verify_manifest(bundle_dir: Path, include_model: bool) -> None:
    """Reference checks (``tasft_model.py:458-498``) for the files this loader reads."""
    manifest_path = bundle_dir / "manifest.json"
    if not manifest_path.exists():
        raise BundleError("manifest.json not found in bundle", context={"bundle_path": str(bundle_dir)})
    manifest = json.loads(manifest_path.read_text())
    checksums: dict[str, str] = manifest.get("checksums", {})
    if not checksums:
        raise BundleError("No checksums found in manifest", context={"bundle_path": str(bundle_dir)})
    for rel, expected in checksums.items():
        if rel.startswith("model/") and not include_model:
            continue
        path = bundle_dir / rel
        if not path.exists():
            raise BundleError(f"File listed in manifest not found: {rel}",
                              context={"relative_path": rel, "bundle_path": str(bundle_dir)})
        actual = _sha256(path)
        if actual != expected:
            raise ChecksumError(f"Checksum mismatch for {path.name}",
                                context={"path": str(path), "expected": expected, "actual": actual})


def load_bundle_gates(bundle_dir: str | Path, num_heads: int, head_dim: int, *,
                      device: str | torch.device = "cpu", dtype: torch.dtype = torch.float32,
                      verify: str = "gates") -> BundleGates:
    """Load every ``gates/layer_{i}_gate.safetensors`` of a bundle as an ``AttnGate``.

    Args:
        bundle_dir: the bundle directory.
        num_heads, head_dim: the attention geometry (the reference reads them from the
            model's first attention layer).
        device, dtype: where the gates live (the reference casts them to the model dtype).
        verify: ``"gates"`` checks the manifest checksums of the gate files and
            ``kernel_config.json``; ``"all"`` also those of ``model/``; ``"none"`` skips.

    Raises:
        BundleError: missing directory, file or manifest entry; a state dict that does not
            fit ``(num_heads, head_dim)`` or the config's ``gate_hidden_dim``.
        ChecksumError: a file whose SHA-256 differs from the manifest.
    """
    bundle_dir = Path(bundle_dir)
    if not bundle_dir.is_dir():
        raise BundleError("Bundle path is not a directory", context={"path": str(bundle_dir)})
    if verify not in ("gates", "all", "none"):
        raise ValueError(f"verify must be 'gates', 'all' or 'none', got {verify!r}")
    if verify != "none":
        _verify_manifest(bundle_dir, include_model=verify == "all")
    gates_dir = bundle_dir / "gates"
    if not gates_dir.is_dir():
        raise BundleError("gates/ subdirectory not found in bundle", context={"bundle_path": str(bundle_dir)})
    cfg_path = bundle_dir / "kernel_config.json"
    if not cfg_path.exists():
        raise BundleError("kernel_config.json not found in bundle", context={"bundle_path": str(bundle_dir)})
    kernel_config = KernelConfig(**json.loads(cfg_path.read_text()))

    from safetensors.torch import load_file

    layers = sorted(int(m.group(1)) for f in gates_dir.iterdir() if (m := _GATE_FILE.match(f.name)))
    if not layers:
        raise BundleError("No gate files in gates/", context={"gates_dir": str(gates_dir)})
    gates: dict[int, AttnGate] = {}
    thresholds: dict[int, float | torch.Tensor] = {}
    block_sizes: dict[int, int] = {}
    for i in layers:
        state = load_file(str(gates_dir / f"layer_{i}_gate.safetensors"))
        w = state.get("gate_proj_in.weight")
        if w is None or w.ndim != 2 or w.shape[1] != 2 * head_dim:
            raise BundleError(
                f"Layer {i} gate state does not fit head_dim={head_dim}",
                context={"layer_idx": i, "gate_proj_in.weight": list(w.shape) if w is not None else None})
        hidden = int(w.shape[0])
        layer_cfg = kernel_config.per_layer_config.get(i)
        if layer_cfg is not None and layer_cfg.gate_hidden_dim is not None and layer_cfg.gate_hidden_dim != hidden:
            raise BundleError(
                f"Layer {i} gate has hidden width {hidden}, kernel_config says {layer_cfg.gate_hidden_dim}",
                context={"layer_idx": i, "state": hidden, "config": layer_cfg.gate_hidden_dim})
        bs = kernel_config.get_layer_block_size(i)
        gate = AttnGate(num_heads=num_heads, head_dim=head_dim, block_size=bs, gate_hidden_dim=hidden)
        gate.load_state_dict(state)
        gate = gate.to(device=device, dtype=dtype).eval().requires_grad_(False)
        gates[i] = gate
        block_sizes[i] = bs
        if layer_cfg is not None and layer_cfg.threshold_tau_per_head is not None:
            taus = kernel_config.get_layer_head_thresholds(i, num_heads)
            thresholds[i] = torch.tensor(taus, dtype=torch.float32, device=device)
        else:
            thresholds[i] = kernel_config.get_layer_threshold(i)
    return BundleGates(gates=gates, thresholds=thresholds, block_sizes=block_sizes,
                       kernel_config=kernel_config)


__all__ = ["BundleGates", "load_bundle_gates"]
