"""Inference side of the hot path: cached sparse decoding (the gate-driven decode step
the reference does not define) and the gates of a TASFT bundle."""
from tasft_amd.inference.bundle_gates import BundleGates, load_bundle_gates
from tasft_amd.inference.sparse_decode import SparseAttentionDecoder

__all__ = ["BundleGates", "SparseAttentionDecoder", "load_bundle_gates"]
