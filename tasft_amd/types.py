"""Shared constants and tensor aliases (reference: ``tasft/types.py:12-27``)."""
from __future__ import annotations

from typing import Final, NewType, TypeAlias

import torch

# Block sizes the attention kernels accept (reference ``tasft/types.py:12``).
VALID_BLOCK_SIZES: Final[frozenset[int]] = frozenset({32, 64, 128})

BlockMask: TypeAlias = torch.Tensor  # [B, H, NB_q, NB_k] bool
AttentionScores: TypeAlias = torch.Tensor  # [B, H, S, S] float
SoftGateScores: TypeAlias = torch.Tensor  # [B, H, NB_q, NB_k] float in [0, 1]
BlockImportance: TypeAlias = torch.Tensor  # [B, H, NB_q, NB_k] float
LayerIndex = NewType("LayerIndex", int)
SparsityRatio = NewType("SparsityRatio", float)

__all__ = [
    "VALID_BLOCK_SIZES",
    "AttentionScores",
    "BlockImportance",
    "BlockMask",
    "LayerIndex",
    "SoftGateScores",
    "SparsityRatio",
]
