"""Cached sparse decoding (the gate-driven decode step the reference does not define)."""
from tasft_amd.inference.sparse_decode import SparseAttentionDecoder

__all__ = ["SparseAttentionDecoder"]
