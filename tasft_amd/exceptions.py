"""Exception hierarchy of the block-sparse attention path.

Same class names, parentage and ``context`` attribute as the reference
(``tasft/exceptions.py:7-44``) so callers that catch ``KernelError`` or
``ValidationError`` keep working unchanged.
"""
from __future__ import annotations

from typing import Any


class TASFTError(Exception):
    """Base error; carries a structured ``context`` dict for logging."""

    def __init__(self, message: str, context: dict[str, Any] | None = None) -> None:
        super().__init__(message)
        self.context: dict[str, Any] = context or {}


class TrainingError(TASFTError):
    """Unrecoverable training-side error."""


class NaNDetectedError(TrainingError):
    """NaN or +inf found where finite values are required."""


class OOMError(TrainingError):
    """Out of memory with no recovery."""


class InferenceError(TASFTError):
    """Inference-time error."""


class BundleError(TASFTError):
    """Bundle export/import error."""


class ChecksumError(BundleError):
    """Checksum mismatch."""


class ValidationError(TASFTError):
    """Invalid input (shapes, ranges)."""


class KernelError(TASFTError):
    """Sparse attention kernel error: bad shape, device, dtype or launch failure."""


__all__ = [
    "BundleError",
    "ChecksumError",
    "InferenceError",
    "KernelError",
    "NaNDetectedError",
    "OOMError",
    "TASFTError",
    "TrainingError",
    "ValidationError",
]
