"""MI355X (gfx950) block-sparse attention hot path of TASFT.

Host code on PyTorch-ROCm calling hand-written HIP kernels through the C ABI of
``tasft_amd/_lib/libtasft_amd.so`` (declared in ``include/tasft_amd.h``).
"""
__version__ = "0.1.0"
__all__ = ["__version__"]
