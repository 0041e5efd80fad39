"""Per-layer kernel configuration (reference: ``tasft/kernels/kernel_config.py:29-171``).

Immutable pydantic models holding the gate threshold and block size per layer.
Field names, validation ranges and error texts follow the reference so a
``kernel_config.json`` written for the reference loads here unchanged.
"""
from __future__ import annotations

from pydantic import BaseModel, ConfigDict, field_validator, model_validator

from tasft_amd.types import VALID_BLOCK_SIZES


def _check_block_size(v: int) -> int:
    if v not in VALID_BLOCK_SIZES:
        msg = f"block_size must be one of {sorted(VALID_BLOCK_SIZES)}, got {v}"
        raise ValueError(msg)
    return v


class LayerKernelConfig(BaseModel):
    """Threshold and block size of one transformer layer (reference ``kernel_config.py:29-72``).

    Optional additions (absent in a reference file, so those load unchanged):

    * ``gate_loss_validation``: the field the reference exporter writes for every layer
      (``tasft/bundle/bundle_schema.py:42``) but its loader's model forbids, so an exported
      bundle's ``kernel_config.json`` failed to load there; accepted here.
    * ``threshold_tau_per_head``: one threshold per query head, each in (0, 1); the gate
      takes them as its per-head ``threshold`` tensor.
    * ``gate_hidden_dim``: the AttnGate hidden width the layer was trained with (the
      reference loader always builds the default width, ``tasft/bundle/tasft_model.py:570-574``).
    """

    model_config = ConfigDict(frozen=True, extra="forbid")

    layer_idx: int
    threshold_tau: float
    target_sparsity: float
    achieved_sparsity_validation: float
    block_size: int = 64
    gate_loss_validation: float | None = None
    threshold_tau_per_head: tuple[float, ...] | None = None
    gate_hidden_dim: int | None = None

    @field_validator("threshold_tau_per_head")
    @classmethod
    def _validate_per_head(cls, v: tuple[float, ...] | None) -> tuple[float, ...] | None:
        if v is None:
            return v
        if len(v) == 0:
            msg = "threshold_tau_per_head must not be empty"
            raise ValueError(msg)
        for i, t in enumerate(v):
            if not 0.0 < t < 1.0:
                msg = f"threshold_tau_per_head[{i}] must be in (0, 1), got {t}"
                raise ValueError(msg)
        return v

    @field_validator("gate_hidden_dim")
    @classmethod
    def _validate_hidden(cls, v: int | None) -> int | None:
        if v is not None and v <= 0:
            msg = f"gate_hidden_dim must be positive, got {v}"
            raise ValueError(msg)
        return v

    @field_validator("threshold_tau")
    @classmethod
    def _validate_threshold(cls, v: float) -> float:
        if not 0.0 < v < 1.0:
            msg = f"threshold_tau must be in (0, 1), got {v}"
            raise ValueError(msg)
        return v

    @field_validator("target_sparsity", "achieved_sparsity_validation")
    @classmethod
    def _validate_sparsity(cls, v: float) -> float:
        if not 0.0 <= v <= 1.0:
            msg = f"sparsity must be in [0, 1], got {v}"
            raise ValueError(msg)
        return v

    @field_validator("block_size")
    @classmethod
    def _validate_block_size(cls, v: int) -> int:
        return _check_block_size(v)


class KernelConfig(BaseModel):
    """Global defaults plus per-layer overrides (reference ``kernel_config.py:75-171``)."""

    model_config = ConfigDict(frozen=True, extra="forbid")

    block_size: int = 64
    global_threshold: float = 0.5
    per_layer_config: dict[int, LayerKernelConfig] = {}
    min_sparsity_for_speedup: float = 0.5

    @field_validator("global_threshold")
    @classmethod
    def _validate_threshold(cls, v: float) -> float:
        if not 0.0 < v < 1.0:
            msg = f"global_threshold must be in (0, 1), got {v}"
            raise ValueError(msg)
        return v

    @field_validator("block_size")
    @classmethod
    def _validate_block_size(cls, v: int) -> int:
        return _check_block_size(v)

    @field_validator("min_sparsity_for_speedup")
    @classmethod
    def _validate_min_sparsity(cls, v: float) -> float:
        if not 0.0 <= v <= 1.0:
            msg = f"min_sparsity_for_speedup must be in [0, 1], got {v}"
            raise ValueError(msg)
        return v

    @model_validator(mode="after")
    def _validate_layer_consistency(self) -> KernelConfig:
        for layer_idx, cfg in self.per_layer_config.items():
            if cfg.layer_idx != layer_idx:
                msg = f"Layer config key {layer_idx} doesn't match cfg.layer_idx {cfg.layer_idx}"
                raise ValueError(msg)
            if cfg.block_size != self.block_size:
                msg = f"Layer {layer_idx} block_size {cfg.block_size} != global {self.block_size}"
                raise ValueError(msg)
        return self

    def get_layer_threshold(self, layer_idx: int) -> float:
        """Threshold of ``layer_idx``, else the global one (reference ``kernel_config.py:142-155``)."""
        if layer_idx in self.per_layer_config:
            return self.per_layer_config[layer_idx].threshold_tau
        return self.global_threshold

    def get_layer_head_thresholds(self, layer_idx: int, num_heads: int) -> tuple[float, ...]:
        """Per-head thresholds of ``layer_idx`` (``num_heads`` copies of the scalar one when the
        layer has none), for ``AttnGate.forward(threshold=torch.tensor(...))``."""
        cfg = self.per_layer_config.get(layer_idx)
        if cfg is not None and cfg.threshold_tau_per_head is not None:
            if len(cfg.threshold_tau_per_head) != num_heads:
                msg = (f"Layer {layer_idx} has {len(cfg.threshold_tau_per_head)} per-head "
                       f"thresholds, expected {num_heads}")
                raise ValueError(msg)
            return cfg.threshold_tau_per_head
        return (self.get_layer_threshold(layer_idx),) * num_heads

    def get_layer_block_size(self, layer_idx: int) -> int:
        """Block size of ``layer_idx``, else the global one (reference ``kernel_config.py:157-170``)."""
        if layer_idx in self.per_layer_config:
            return self.per_layer_config[layer_idx].block_size
        return self.block_size


__all__ = ["KernelConfig", "LayerKernelConfig"]
