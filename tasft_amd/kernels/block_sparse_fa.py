"""Block-sparse flash attention on MI355X (gfx950) behind the reference API.

Mirrors ``tasft.kernels.block_sparse_fa`` (reference ``tasft/kernels/block_sparse_fa.py:54-618``):
same class, constructor, ``forward`` signature, validation order and messages, sparsity
statistics and low-sparsity policy. The compute backend is the hand-written HIP library
``libtasft_amd.so`` reached through its C ABI; there is no Triton and no second kernel
backend. ``DENSE_FALLBACK`` stays what it is in the reference: torch SDPA, which ignores
the block mask, used only when explicitly requested or when the mask is denser than
``min_sparsity_for_speedup`` (reference ``:392-399``).

Additive, keyword-compatible extensions:
  * GQA-native ``forward``: ``k``/``v`` may carry ``Hkv`` heads with ``Hq % Hkv == 0``
    (query head ``h`` reads KV head ``h // (Hq // Hkv)``, the ``repeat_interleave``
    mapping of ``tasft/modules/tasft_attention.py:725-729``), so callers no longer
    expand K/V.
  * ``forward_decode``: split-K block-sparse decode for one new token per sequence.
"""
from __future__ import annotations

import math
import warnings
from dataclasses import dataclass
from enum import Enum, auto

import torch
from torch.nn import functional

from tasft_amd import _native
from tasft_amd.exceptions import KernelError
from tasft_amd.types import VALID_BLOCK_SIZES

_VALID_HEAD_DIMS = frozenset({64, 128})
_EXPECTED_TENSOR_NDIM = 4


class KernelBackend(Enum):
    """Backends of the reference enum plus the gfx950 HIP backend.

    ``FLASH_ATTN_SPARSE`` and ``TRITON`` are kept so reference code that names them still
    imports; they are never available here. ``HIP_GFX950`` is the only compute backend.
    """

    AUTO = auto()
    FLASH_ATTN_SPARSE = auto()
    TRITON = auto()
    HIP_GFX950 = auto()
    DENSE_FALLBACK = auto()


def detect_kernels() -> list[KernelBackend]:
    """Available backends, highest priority first; ``DENSE_FALLBACK`` is always last.

    Reference: ``block_sparse_fa.py:63-90``. Probes only whether the C-ABI library loads;
    it never touches the GPU.
    """
    available: list[KernelBackend] = []
    if _native.is_available():
        available.append(KernelBackend.HIP_GFX950)
    available.append(KernelBackend.DENSE_FALLBACK)
    return available


@dataclass(frozen=True, slots=True)
class SparsityStats:
    """Block-mask statistics (reference ``block_sparse_fa.py:277-291``).

    ``sparsity_ratio`` counts the full NB x NB grid, upper triangle included, exactly as
    the reference does (``:586-588``).
    """

    total_blocks: int
    active_blocks: int
    sparsity_ratio: float
    estimated_speedup: float


def _kv_compatible(q: torch.Tensor, kv: torch.Tensor) -> bool:
    if kv.ndim != _EXPECTED_TENSOR_NDIM:
        return False
    b, hq, s, d = q.shape
    bk, hk, sk, dk = kv.shape
    return bk == b and sk == s and dk == d and hk > 0 and hq % hk == 0


def _kernel_dtype(**tensors: torch.Tensor) -> int:
    """The C-ABI ``dtype`` code shared by the given tensors (bf16 or fp16, all the same, as the
    reference's ``tl.dot`` needs, ``block_sparse_fa.py:228, 252``)."""
    items = list(tensors.items())
    first_name, first = items[0]
    for name, t in items[1:]:
        if t.dtype != first.dtype:
            raise KernelError(f"{name} is {t.dtype} but {first_name} is {first.dtype}",
                              context={"tensor": name, "dtype": str(t.dtype), "expected": str(first.dtype)})
    return _native.dtype_code(first.dtype, "block-sparse attention")


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` if its layout suits the kernels (unit d stride, 16-byte rows), else a copy."""
    st = t.stride()
    if st[-1] == 1 and all(s % 8 == 0 for s in st[:-1]) and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def _mask_bytes(mask: torch.Tensor) -> torch.Tensor:
    """One byte per block, non-zero = attend, without a copy for bool masks."""
    if mask.dtype == torch.bool:
        return mask.view(torch.uint8)
    if mask.dtype in (torch.uint8, torch.int8):
        return mask.view(torch.uint8) if mask.dtype == torch.int8 else mask
    return (mask != 0).view(torch.uint8)


class BlockSparseFlashAttention:
    """Block-sparse flash attention with the reference constructor and ``forward``.

    Args:
        block_size: Attention block granularity in tokens; one of {32, 64, 128}.
        min_sparsity_for_speedup: Below this mask sparsity (full-grid count), ``forward``
            warns and returns dense SDPA, ignoring the mask (reference behaviour).
        backend: ``AUTO`` or ``HIP_GFX950`` (the HIP kernels), or ``DENSE_FALLBACK``.

    Raises:
        ValueError: ``block_size`` or ``min_sparsity_for_speedup`` out of range.
        KernelError: the requested backend is not available.
    """

    def __init__(
        self,
        block_size: int = 64,
        min_sparsity_for_speedup: float = 0.5,
        backend: KernelBackend = KernelBackend.AUTO,
    ) -> None:
        if block_size not in VALID_BLOCK_SIZES:
            raise ValueError(
                f"block_size must be one of {sorted(VALID_BLOCK_SIZES)}, got {block_size}"
            )
        if not 0.0 <= min_sparsity_for_speedup <= 1.0:
            raise ValueError(
                f"min_sparsity_for_speedup must be in [0, 1], got {min_sparsity_for_speedup}"
            )
        self.block_size = block_size
        self.min_sparsity_for_speedup = min_sparsity_for_speedup
        self._available_backends = detect_kernels()
        if backend == KernelBackend.AUTO:
            # The HIP backend is selected even if the library is absent, so a missing
            # build surfaces as a KernelError at the first forward instead of a silent
            # switch to dense attention.
            self.backend = KernelBackend.HIP_GFX950
        elif backend in (KernelBackend.HIP_GFX950, KernelBackend.DENSE_FALLBACK):
            self.backend = backend
        else:
            available_names = [b.name for b in self._available_backends]
            msg = f"Requested backend {backend.name} is not available. Available: {available_names}"
            raise KernelError(msg, context={"requested": backend.name, "available": available_names})

    # ------------------------------------------------------------------ prefill
    def forward(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        block_mask: torch.Tensor,
        *,
        causal: bool = True,
    ) -> torch.Tensor:
        """Block-sparse attention ``[B, Hq, S, D]`` (reference ``block_sparse_fa.py:361-411``).

        ``k``/``v`` are ``[B, Hkv, S, D]`` with ``Hq % Hkv == 0`` (``Hkv == Hq`` is the
        reference case). ``block_mask`` is ``[B, Hq, NB, NB]``; with ``causal`` it is
        AND-ed with the block lower triangle and the diagonal blocks are masked
        element-wise. Rows with no active block are zero.
        """
        self._validate_inputs(q, k, v, block_mask)
        if self.min_sparsity_for_speedup > 0.0:
            # The statistics need a device->host sync; with a 0.0 threshold the
            # comparison below can never fire, so it is skipped.
            stats = self.compute_sparsity_stats(block_mask)
            if stats.sparsity_ratio < self.min_sparsity_for_speedup:
                warnings.warn(
                    f"Sparsity {stats.sparsity_ratio:.2%} below threshold "
                    f"{self.min_sparsity_for_speedup:.2%}; using dense fallback.",
                    stacklevel=2,
                )
                return self._dense_fallback(q, k, v, causal)
        if self.backend == KernelBackend.DENSE_FALLBACK:
            return self._dense_fallback(q, k, v, causal)
        return self._hip_forward(q, k, v, block_mask, causal)

    __call__ = forward

    def _validate_inputs(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        block_mask: torch.Tensor,
    ) -> None:
        """Reference checks and messages (``block_sparse_fa.py:413-452``), GQA-aware."""
        if q.ndim != _EXPECTED_TENSOR_NDIM:
            msg = f"Expected 4D tensors [B, H, S, D], got q.ndim={q.ndim}"
            raise KernelError(msg, context={"q_shape": list(q.shape)})
        if k.shape != v.shape or not _kv_compatible(q, k):
            raise KernelError(
                "Q, K, V shapes must match",
                context={"q": list(q.shape), "k": list(k.shape), "v": list(v.shape)},
            )
        if not q.is_cuda:
            raise KernelError("Tensors must be on CUDA device", context={"device": str(q.device)})
        B, H, S, _D = q.shape
        num_blocks = math.ceil(S / self.block_size)
        expected_mask_shape = (B, H, num_blocks, num_blocks)
        if tuple(block_mask.shape) != expected_mask_shape:
            raise KernelError(
                f"block_mask shape mismatch: expected {expected_mask_shape}, "
                f"got {tuple(block_mask.shape)}",
                context={
                    "expected": list(expected_mask_shape),
                    "got": list(block_mask.shape),
                    "block_size": self.block_size,
                },
            )

    def _hip_forward(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        block_mask: torch.Tensor,
        causal: bool,
    ) -> torch.Tensor:
        """Launch ``tasft_bsfa_prefill_fwd`` on the current stream (replaces ``:454-552``)."""
        B, H, S, D = q.shape
        if D not in _VALID_HEAD_DIMS:
            raise KernelError(
                f"HIP kernel supports head_dim in {sorted(_VALID_HEAD_DIMS)}, got {D}",
                context={"head_dim": D, "supported": sorted(_VALID_HEAD_DIMS)},
            )
        dtype = _kernel_dtype(q=q, k=k, v=v)
        for t in (k, v):
            if t.device != q.device:
                raise KernelError("Q, K, V must be on the same device", context={"device": str(t.device)})
        lib = _native.load_library()
        q = _kernel_ready(q)
        k = _kernel_ready(k)
        v = _kernel_ready(v)
        mask = _mask_bytes(block_mask.to(q.device))
        out = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
        scale = 1.0 / math.sqrt(D)
        # Workspace for the persistent launch's work-queue counters.
        ws_bytes = lib.tasft_bsfa_prefill_workspace_bytes(B, H, S, self.block_size)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        status = lib.tasft_bsfa_prefill_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), mask.data_ptr(),
            workspace.data_ptr(), ws_bytes, B, H, k.shape[1], S, D, self.block_size,
            _native.strides(q), _native.strides(k), _native.strides(v), _native.strides(out),
            _native.strides(mask), scale, 1 if causal else 0, dtype, _native.stream_handle(q.device),
        )
        _native.check(status, "tasft_bsfa_prefill_fwd", {"shape": [B, H, S, D]})
        return out

    def _dense_fallback(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        causal: bool,
    ) -> torch.Tensor:
        """Dense SDPA ignoring the mask (reference ``block_sparse_fa.py:554-572``)."""
        gqa = k.shape[1] != q.shape[1]
        return functional.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=gqa)

    # ------------------------------------------------------------------ varlen prefill
    def forward_varlen(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        block_mask: torch.Tensor,
        cu_seqlens: torch.Tensor,
        max_seqlen: int | None = None,
        *,
        causal: bool = True,
    ) -> torch.Tensor:
        """Block-sparse prefill of a packed batch of variable-length sequences (one launch).

        The reference's vLLM backend views all packed tokens as one sequence
        (``tasft/inference/vllm_patch.py:172-176``), so a request also attends to the
        requests packed before it; here each sequence attends only within itself, with the
        semantics of ``forward`` per sequence. There is no low-sparsity dense fallback.

        Args:
            q: ``[T, Hq, D]`` packed queries; k, v: ``[T, Hkv, D]``, ``Hq % Hkv == 0``; all
                bf16 or all fp16.
            block_mask: ``[N, Hq, NB, NB]`` with ``NB = ceil(max_seqlen / block_size)``;
                sequence n uses its leading ``ceil(len_n / block_size)`` square.
            cu_seqlens: ``[N + 1]`` int32 cumulative lengths (``cu_seqlens[0] == 0``,
                non-decreasing, ``cu_seqlens[N] <= T``). On the CPU it is checked here and
                copied to the device; on the device it is trusted (no synchronisation),
                and ``max_seqlen`` must be given.
            max_seqlen: the longest sequence (default: from a CPU ``cu_seqlens``).
            causal: causal masking within each sequence.

        Returns:
            ``[T, Hq, D]``; rows of tokens after ``cu_seqlens[N]`` are 0.
        """
        if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
            raise KernelError(
                "Expected packed q, k, v of shape [T, H, D]",
                context={"q_shape": list(q.shape), "k_shape": list(k.shape), "v_shape": list(v.shape)},
            )
        T, H, D = q.shape
        if k.shape != v.shape or k.shape[0] != T or k.shape[2] != D or k.shape[1] <= 0 or H % k.shape[1] != 0:
            raise KernelError(
                f"K/V must be [T, Hkv, D] with Hq % Hkv == 0; got q {tuple(q.shape)}, "
                f"k {tuple(k.shape)}, v {tuple(v.shape)}",
                context={"q_shape": list(q.shape), "k_shape": list(k.shape), "v_shape": list(v.shape)},
            )
        if D not in _VALID_HEAD_DIMS:
            raise KernelError(
                f"HIP kernel supports head_dim in {sorted(_VALID_HEAD_DIMS)}, got {D}",
                context={"head_dim": D, "supported": sorted(_VALID_HEAD_DIMS)},
            )
        if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
            raise KernelError("cu_seqlens must be a 1-D tensor of N + 1 >= 2 offsets",
                              context={"cu_seqlens_shape": list(cu_seqlens.shape)})
        n_seq = cu_seqlens.numel() - 1
        if cu_seqlens.device.type == "cpu":
            cu = cu_seqlens.to(torch.int64)
            lens = cu[1:] - cu[:-1]
            if int(cu[0]) != 0 or bool((lens < 0).any()) or int(cu[-1]) > T:
                raise KernelError(
                    "cu_seqlens must start at 0, be non-decreasing and end at <= T",
                    context={"cu_seqlens": cu.tolist()[:16], "T": T},
                )
            longest = int(lens.max())
            if max_seqlen is None:
                max_seqlen = max(longest, 1)
            elif longest > max_seqlen:
                raise KernelError(
                    f"a sequence has {longest} tokens, more than max_seqlen={max_seqlen}",
                    context={"max_seqlen": max_seqlen, "longest": longest},
                )
            covered = int(cu[-1])
        else:
            if max_seqlen is None:
                raise KernelError("max_seqlen is required when cu_seqlens is on the device",
                                  context={"device": str(cu_seqlens.device)})
            covered = -1  # unknown without a synchronisation
        if max_seqlen <= 0:
            raise KernelError(f"max_seqlen must be positive, got {max_seqlen}",
                              context={"max_seqlen": max_seqlen})
        nb = math.ceil(max_seqlen / self.block_size)
        expected = (n_seq, H, nb, nb)
        if tuple(block_mask.shape) != expected:
            raise KernelError(
                f"block_mask shape mismatch: expected {expected}, got {tuple(block_mask.shape)}",
                context={"expected": list(expected), "got": list(block_mask.shape)},
            )
        dtype = _kernel_dtype(q=q, k=k, v=v)
        for name, t in (("q", q), ("k", k), ("v", v)):
            if not t.is_cuda or t.device != q.device:
                raise KernelError("Q, K, V must be on the same GPU device",
                                  context={"tensor": name, "device": str(t.device)})
        lib = _native.load_library()
        q = _kernel_ready(q)
        k = _kernel_ready(k)
        v = _kernel_ready(v)
        mask = _mask_bytes(block_mask.to(q.device))
        cu_dev = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
        out = torch.empty_like(q)
        status = lib.tasft_bsfa_prefill_varlen_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), mask.data_ptr(),
            cu_dev.data_ptr(), n_seq, H, k.shape[1], max_seqlen, D, self.block_size,
            _native.strides(q), _native.strides(k), _native.strides(v), _native.strides(out),
            _native.strides(mask), 1.0 / math.sqrt(D), 1 if causal else 0, dtype,
            _native.stream_handle(q.device),
        )
        _native.check(status, "tasft_bsfa_prefill_varlen_fwd",
                      {"tokens": T, "sequences": n_seq, "max_seqlen": max_seqlen})
        if covered != T:
            # Rows no sequence covers are zeroed on the device (cu_seqlens[N] is read there,
            # so a device cu_seqlens needs no host round trip).
            status = lib.tasft_bsfa_varlen_zero_tail(
                out.data_ptr(), cu_dev.data_ptr(), n_seq, T, H, D, _native.strides(out),
                _native.stream_handle(q.device))
            _native.check(status, "tasft_bsfa_varlen_zero_tail", {"tokens": T, "sequences": n_seq})
        return out

    # ------------------------------------------------------------------ decode
    def forward_decode(
        self,
        q: torch.Tensor,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        block_mask: torch.Tensor | None = None,
        *,
        block_indices: torch.Tensor | None = None,
        kv_lens: torch.Tensor | None = None,
        num_splits: int | None = None,
    ) -> torch.Tensor:
        """Block-sparse decode of one new token per sequence.

        Args:
            q: ``[B, Hq, 1, D]``, the new token's queries (bf16 or fp16).
            k_cache, v_cache: ``[B, Hkv, S_kv, D]`` of q's dtype; the new token's K/V are
                included.
            block_mask: ``[B, Hq, 1, ceil(S_kv / block_size)]``; non-zero selects a block.
            block_indices: instead of ``block_mask``, ``[B, Hq, K]`` integer lists of the
                selected block indices per head, ``-1`` marking empty slots (converted on
                the GPU by ``tasft_mask_from_indices``; duplicates are harmless).
            kv_lens: optional ``[B]`` int32 valid lengths (default ``S_kv``).
            num_splits: split-K factor (default: sized so the launch fills the GPU).

        Returns:
            ``[B, Hq, 1, D]``: ``softmax(q K_sel^T / sqrt(D)) V_sel`` per head, 0 for a head
            with no selected block. There is no reference counterpart: reference decode is
            dense (``tasft/inference/vllm_patch.py:189-196``).
        """
        if q.ndim != _EXPECTED_TENSOR_NDIM or q.shape[2] != 1:
            raise KernelError(
                f"Expected q of shape [B, H, 1, D], got {tuple(q.shape)}",
                context={"q_shape": list(q.shape)},
            )
        if (
            k_cache.ndim != _EXPECTED_TENSOR_NDIM
            or k_cache.shape != v_cache.shape
            or k_cache.shape[0] != q.shape[0]
            or k_cache.shape[3] != q.shape[3]
            or q.shape[1] % k_cache.shape[1] != 0
        ):
            raise KernelError(
                "KV cache shape incompatible with q",
                context={"q": list(q.shape), "k": list(k_cache.shape), "v": list(v_cache.shape)},
            )
        if not q.is_cuda:
            raise KernelError("Tensors must be on CUDA device", context={"device": str(q.device)})
        B, H, _, D = q.shape
        Hkv, S_kv = k_cache.shape[1], k_cache.shape[2]
        nb = math.ceil(S_kv / self.block_size)
        if (block_mask is None) == (block_indices is None):
            raise KernelError("Pass exactly one of block_mask and block_indices",
                              context={"block_mask": block_mask is not None,
                                       "block_indices": block_indices is not None})
        if block_indices is not None:
            if block_indices.ndim != 3 or tuple(block_indices.shape[:2]) != (B, H):
                raise KernelError(
                    f"block_indices must have shape [{B}, {H}, K], got {tuple(block_indices.shape)}",
                    context={"expected": [B, H, -1], "got": list(block_indices.shape)},
                )
            block_mask = indices_to_mask(block_indices.to(q.device), nb).view(B, H, 1, nb)
        if tuple(block_mask.shape) != (B, H, 1, nb):
            raise KernelError(
                f"block_mask shape mismatch: expected {(B, H, 1, nb)}, got {tuple(block_mask.shape)}",
                context={"expected": [B, H, 1, nb], "got": list(block_mask.shape)},
            )
        if D not in _VALID_HEAD_DIMS:
            raise KernelError(
                f"HIP kernel supports head_dim in {sorted(_VALID_HEAD_DIMS)}, got {D}",
                context={"head_dim": D},
            )
        dtype = _kernel_dtype(q=q, k_cache=k_cache, v_cache=v_cache)
        lib = _native.load_library()
        if num_splits is None:
            # A 128-key block runs as its two 64-key halves: the split counts halves.
            nb_run = math.ceil(S_kv / 64) if self.block_size == 128 else nb
            num_splits = default_decode_splits(B, Hkv, nb_run, H // Hkv)
        q = q.contiguous()
        k_cache = _kernel_ready(k_cache)
        v_cache = _kernel_ready(v_cache)
        mask = _mask_bytes(block_mask.to(q.device))
        lens = None
        if kv_lens is not None:
            lens = kv_lens.to(device=q.device, dtype=torch.int32).contiguous()
            if lens.shape != (B,):
                raise KernelError(f"kv_lens must have shape ({B},), got {tuple(lens.shape)}",
                                  context={"kv_lens": list(lens.shape)})
        ws_bytes = lib.tasft_bsfa_decode_workspace_bytes(B, H, D, num_splits)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        out = torch.empty((B, H, 1, D), dtype=q.dtype, device=q.device)
        status = lib.tasft_bsfa_decode_fwd(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), mask.data_ptr(),
            _native.ptr(lens), workspace.data_ptr(), ws_bytes, B, H, Hkv, S_kv, D,
            self.block_size, num_splits,
            _native.strides(q), _native.strides(k_cache), _native.strides(v_cache),
            _native.strides(out), _native.strides(mask), 1.0 / math.sqrt(D), dtype,
            _native.stream_handle(q.device),
        )
        _native.check(status, "tasft_bsfa_decode_fwd", {"shape": [B, H, S_kv, D]})
        return out

    # ------------------------------------------------------------------ stats
    def forward_decode_paged(
        self,
        q: torch.Tensor,
        k_pages: torch.Tensor,
        v_pages: torch.Tensor,
        block_table: torch.Tensor,
        kv_lens: torch.Tensor,
        block_mask: torch.Tensor | None = None,
        *,
        block_indices: torch.Tensor | None = None,
        num_splits: int | None = None,
    ) -> torch.Tensor:
        """Block-sparse decode over a paged KV cache (vLLM's block-table layout).

        The reference hands paged decode to vLLM's dense PagedAttention
        (``tasft/inference/vllm_patch.py:189-196, 215-252``); this reads only the selected
        key blocks, through the block table, with the result of ``forward_decode`` on the
        equivalent contiguous cache.

        Args:
            q: ``[B, Hq, 1, D]`` (bf16 or fp16).
            k_pages, v_pages: ``[num_pages, page_size, Hkv, D]`` page pools of q's dtype; token t of
                sequence b is row ``t % page_size`` of page ``block_table[b, t // page_size]``.
            block_table: ``[B, max_pages]`` int32 on the device; only the pages holding a
                token below ``kv_lens[b]`` are read. An entry outside
                ``[0, num_pages)`` is clamped into it by the kernel (wrong values, never an
                access outside the pools).
            kv_lens: ``[B]`` int32 valid lengths (on the device).
            block_mask: ``[B, Hq, 1, NB]`` with ``NB = ceil(max_pages * page_size / block_size)``.
            block_indices: instead of ``block_mask``, ``[B, Hq, K]`` index lists (``-1`` empty).
            num_splits: split-K factor (default: sized so the launch fills the GPU).

        Returns:
            ``[B, Hq, 1, D]``.
        """
        if q.ndim != _EXPECTED_TENSOR_NDIM or q.shape[2] != 1:
            raise KernelError(f"Expected q of shape [B, H, 1, D], got {tuple(q.shape)}",
                              context={"q_shape": list(q.shape)})
        B, H, _, D = q.shape
        if (
            k_pages.ndim != _EXPECTED_TENSOR_NDIM
            or k_pages.shape != v_pages.shape
            or k_pages.shape[3] != D
            or H % k_pages.shape[2] != 0
        ):
            raise KernelError(
                "page pools must be [num_pages, page_size, Hkv, D] with Hq % Hkv == 0",
                context={"q": list(q.shape), "k": list(k_pages.shape), "v": list(v_pages.shape)},
            )
        page_size, Hkv = k_pages.shape[1], k_pages.shape[2]
        if block_table.ndim != 2 or block_table.shape[0] != B:
            raise KernelError(f"block_table must have shape [{B}, max_pages], got {tuple(block_table.shape)}",
                              context={"block_table": list(block_table.shape)})
        if kv_lens.shape != (B,):
            raise KernelError(f"kv_lens must have shape ({B},), got {tuple(kv_lens.shape)}",
                              context={"kv_lens": list(kv_lens.shape)})
        if page_size < 8 or page_size & (page_size - 1):
            raise KernelError(f"page_size must be a power of two >= 8, got {page_size}",
                              context={"page_size": page_size})
        if D not in _VALID_HEAD_DIMS:
            raise KernelError(f"HIP kernel supports head_dim in {sorted(_VALID_HEAD_DIMS)}, got {D}",
                              context={"head_dim": D})
        S_kv = block_table.shape[1] * page_size
        nb = math.ceil(S_kv / self.block_size)
        if (block_mask is None) == (block_indices is None):
            raise KernelError("Pass exactly one of block_mask and block_indices",
                              context={"block_mask": block_mask is not None,
                                       "block_indices": block_indices is not None})
        dtype = _kernel_dtype(q=q, k_pages=k_pages, v_pages=v_pages)
        for name, t in (("q", q), ("k_pages", k_pages), ("v_pages", v_pages)):
            if not t.is_cuda or t.device != q.device:
                raise KernelError("Tensors must be on one CUDA device",
                                  context={"tensor": name, "device": str(t.device)})
        if block_indices is not None:
            if block_indices.ndim != 3 or tuple(block_indices.shape[:2]) != (B, H):
                raise KernelError(
                    f"block_indices must have shape [{B}, {H}, K], got {tuple(block_indices.shape)}",
                    context={"expected": [B, H, -1], "got": list(block_indices.shape)},
                )
            block_mask = indices_to_mask(block_indices.to(q.device), nb).view(B, H, 1, nb)
        if tuple(block_mask.shape) != (B, H, 1, nb):
            raise KernelError(
                f"block_mask shape mismatch: expected {(B, H, 1, nb)}, got {tuple(block_mask.shape)}",
                context={"expected": [B, H, 1, nb], "got": list(block_mask.shape)},
            )
        lib = _native.load_library()
        if num_splits is None:
            # A block-128 mask runs on the 64-key kernel (each 128-key block as its halves).
            nb_run = math.ceil(S_kv / 64) if self.block_size == 128 else nb
            num_splits = default_decode_splits(B, Hkv, nb_run, H // Hkv)
        q = q.contiguous()
        k_pages = _kernel_ready(k_pages)
        v_pages = _kernel_ready(v_pages)
        mask = _mask_bytes(block_mask.to(q.device))
        # The kernel reads the table with a unit column stride.
        table = block_table.to(device=q.device, dtype=torch.int32).contiguous()
        lens = kv_lens.to(device=q.device, dtype=torch.int32).contiguous()
        ws_bytes = lib.tasft_bsfa_decode_workspace_bytes(B, H, D, num_splits)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        out = torch.empty((B, H, 1, D), dtype=q.dtype, device=q.device)
        status = lib.tasft_bsfa_decode_paged_fwd(
            q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), out.data_ptr(), mask.data_ptr(),
            table.data_ptr(), lens.data_ptr(), workspace.data_ptr(), ws_bytes, B, H, Hkv, S_kv, D,
            self.block_size, page_size, k_pages.shape[0], num_splits,
            _native.strides(q), _native.strides(k_pages), _native.strides(v_pages),
            _native.strides(out), _native.strides(mask), table.stride(0), 1.0 / math.sqrt(D), dtype,
            _native.stream_handle(q.device),
        )
        _native.check(status, "tasft_bsfa_decode_paged_fwd", {"shape": [B, H, S_kv, D],
                                                              "page_size": page_size})
        return out

    def compute_sparsity_stats(self, block_mask: torch.Tensor) -> SparsityStats:
        """Full-grid statistics (reference ``block_sparse_fa.py:574-595``; syncs the device)."""
        total_blocks = block_mask.numel()
        active_blocks = int(block_mask.sum().item())
        sparsity_ratio = 1.0 - (active_blocks / max(total_blocks, 1))
        return SparsityStats(
            total_blocks=total_blocks,
            active_blocks=active_blocks,
            sparsity_ratio=sparsity_ratio,
            estimated_speedup=self.estimate_speedup(sparsity_ratio),
        )

    @staticmethod
    def estimate_speedup(sparsity_ratio: float) -> float:
        """``1 / max(1e-6, 1 - 0.98 s)``: the reference's model (``block_sparse_fa.py:597-618``)."""
        gate_overhead = 0.02
        denominator = 1.0 - sparsity_ratio * (1.0 - gate_overhead)
        return 1.0 / max(1e-6, denominator)


def indices_to_mask(block_indices: torch.Tensor, num_blocks: int) -> torch.Tensor:
    """Padded block-index lists ``[..., K]`` (``-1`` = empty) -> bool mask ``[..., num_blocks]``.

    Runs ``tasft_mask_from_indices`` on the device; an index outside ``[0, num_blocks)``
    other than ``-1`` raises ``KernelError`` (this reads one device flag).
    """
    if not block_indices.is_cuda:
        raise KernelError("Tensors must be on CUDA device", context={"device": str(block_indices.device)})
    if block_indices.dtype not in (torch.int32, torch.int64, torch.int16, torch.uint8):
        raise KernelError(f"block indices must be integers, got {block_indices.dtype}",
                          context={"dtype": str(block_indices.dtype)})
    lead = tuple(block_indices.shape[:-1])
    k = block_indices.shape[-1]
    idx = block_indices.reshape(-1, k).to(torch.int32).contiguous()
    rows = idx.shape[0]
    mask = torch.empty((rows, num_blocks), dtype=torch.uint8, device=block_indices.device)
    flag = torch.empty((1,), dtype=torch.int32, device=block_indices.device)
    lib = _native.load_library()
    status = lib.tasft_mask_from_indices(idx.data_ptr(), rows, k, k, num_blocks, mask.data_ptr(),
                                         flag.data_ptr(), _native.stream_handle(idx.device))
    _native.check(status, "tasft_mask_from_indices", {"rows": rows, "k": k})
    if int(flag.item()) != 0:
        raise KernelError(f"block index outside [0, {num_blocks}) (other than -1)",
                          context={"num_blocks": num_blocks})
    return mask.view(torch.bool).view(*lead, num_blocks)


def mask_to_csr(block_mask: torch.Tensor, causal: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense block mask ``[B, H, NBq, NBk]`` -> CSR ``(row_ptr [B*H*NBq + 1], col_idx [nnz])``.

    Rows are ``(b, h, query block)`` in row-major order; column indices ascend within a
    row. With ``causal`` only the lower block triangle counts (the kernel-side AND of the
    reference, ``block_sparse_fa.py:502-508``). Runs ``tasft_mask_compact`` on the device
    and reads the total once to trim ``col_idx``.
    """
    if block_mask.ndim != _EXPECTED_TENSOR_NDIM:
        raise KernelError(f"Expected a 4D block mask, got {block_mask.ndim}D",
                          context={"shape": list(block_mask.shape)})
    if not block_mask.is_cuda:
        raise KernelError("Tensors must be on CUDA device", context={"device": str(block_mask.device)})
    B, H, NBq, NBk = block_mask.shape
    mask = _mask_bytes(block_mask)
    rows = B * H * NBq
    lib = _native.load_library()
    ws_bytes = lib.tasft_mask_compact_workspace_bytes(B, H, NBq)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=mask.device)
    row_ptr = torch.empty((rows + 1,), dtype=torch.int32, device=mask.device)
    capacity = rows * (min(NBq, NBk) if causal else NBk)  # a row holds at most this many
    col_idx = torch.empty((max(capacity, 1),), dtype=torch.int32, device=mask.device)
    status = lib.tasft_mask_compact(mask.data_ptr(), B, H, NBq, NBk, _native.strides(mask),
                                    1 if causal else 0, row_ptr.data_ptr(), col_idx.data_ptr(),
                                    capacity, workspace.data_ptr(), ws_bytes,
                                    _native.stream_handle(mask.device))
    _native.check(status, "tasft_mask_compact", {"shape": [B, H, NBq, NBk]})
    nnz = int(row_ptr[-1].item())
    return row_ptr, col_idx[:nnz]


def default_decode_splits(batch: int, num_kv_heads: int, num_blocks: int,
                          q_per_kv: int = 1) -> int:
    """Split-K factor giving about one decode workgroup per CU (256 on MI355X), for every
    head count up to 16 query heads per KV head. Two workgroups fit per CU, but one per CU
    measured fastest: at B=8 with 28/4 heads 8 splits took 20.8 us against 24.6 us for 16,
    at B=8 with 32/8 heads 4 splits took 25.7 us against 27.5 us for 8, and at B=64 with
    28/4 heads one split took 65.8 us against 70.9 us for two. Fewer splits also mean
    fewer blocks scanned twice and, at one split, no combine pass. Never fewer than the
    splits that keep every split within 1024 key blocks."""
    del q_per_kv  # the kernel's occupancy does not depend on the head count
    groups = max(1, batch * num_kv_heads)
    resident = 256
    want = min(max(1, num_blocks // 4), math.ceil(resident / groups))
    return int(max(1, want, math.ceil(num_blocks / 1024)))


def executed_blocks(block_mask: torch.Tensor, causal: bool = True) -> torch.Tensor:
    """Number of (query block, key block) tiles the prefill kernel computes (device tensor)."""
    m = block_mask != 0
    if causal:
        nb = m.shape[-1]
        m = m & torch.ones(nb, nb, dtype=torch.bool, device=m.device).tril()
    return m.sum()


__all__ = [
    "BlockSparseFlashAttention",
    "KernelBackend",
    "SparsityStats",
    "default_decode_splits",
    "detect_kernels",
    "executed_blocks",
    "indices_to_mask",
    "mask_to_csr",
]
