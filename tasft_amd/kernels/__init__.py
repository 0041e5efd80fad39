"""Block-sparse attention kernels (reference package ``tasft/kernels/__init__.py``)."""
from tasft_amd.kernels.block_sparse_fa import (
    BlockSparseFlashAttention,
    KernelBackend,
    SparsityStats,
    default_decode_splits,
    detect_kernels,
    executed_blocks,
    indices_to_mask,
    mask_to_csr,
)
from tasft_amd.kernels.kernel_config import KernelConfig, LayerKernelConfig

__all__ = [
    "BlockSparseFlashAttention",
    "KernelBackend",
    "KernelConfig",
    "LayerKernelConfig",
    "SparsityStats",
    "default_decode_splits",
    "detect_kernels",
    "executed_blocks",
    "indices_to_mask",
    "mask_to_csr",
]
