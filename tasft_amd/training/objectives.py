"""Gate distillation target: softmax of block-max-pooled attention scores.

Two entry points:

* ``TASFTObjective.compute_gate_target(attn_scores, block_size)`` keeps the reference
  API and semantics (``tasft/training/objectives.py:128-185``) for callers that already
  hold a dense ``[B, H, S, S]`` score tensor: NaN/+inf rejection, -inf padding,
  ``max_pool2d``, softmax over the flat block grid.
* ``gate_target_from_qk(q, k, ...)`` is the MI355X kernel path: it takes Q and K and never
  forms the score tensor. The HIP kernel computes each 64x64 block maximum of
  ``Q K^T * scale`` with bf16 or fp16 MFMA (causal: -inf above the diagonal; plus the caller's
  additive ``attention_mask``), then normalises. It replaces the score producer
  ``tasft/modules/tasft_attention.py:426-458`` followed by ``compute_gate_target``;
  ``normalize="row"`` gives the per-row variant and ``temperature``/``clamp`` the variant
  of ``tasft/modules/tasft_attention.py:272-290``.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from tasft_amd import _native
from tasft_amd.exceptions import KernelError, NaNDetectedError

_NORMALIZE = {"flat": 0, "row": 1, "none": 2}


_EPS = 1e-8  # reference objectives.py:39


def _check_finite(tensor: torch.Tensor, name: str) -> None:
    """NaN/Inf guard with the reference's message and context (objectives.py:67-87)."""
    if not bool(torch.isfinite(tensor).all()):
        has_nan = bool(torch.isnan(tensor).any())
        has_inf = bool(torch.isinf(tensor).any())
        raise NaNDetectedError(
            f"Non-finite values detected in {name}: NaN={has_nan}, Inf={has_inf}",
            context={"tensor_name": name, "has_nan": has_nan, "has_inf": has_inf,
                     "shape": list(tensor.shape), "dtype": str(tensor.dtype)},
        )


class TASFTObjective:
    """The gate terms of the reference objective (``tasft/training/objectives.py:128-235``):
    the gate target, the KL gate loss and the sparsity loss. The task loss, the Kahan sums
    and the trainer around them are outside the hot path."""

    @staticmethod
    def compute_gate_target(attn_scores: torch.Tensor, block_size: int) -> torch.Tensor:
        """Reference dense path on a given score tensor (``objectives.py:128-185``)."""
        has_nan = bool(torch.isnan(attn_scores).any())
        has_pos_inf = bool((attn_scores == float("inf")).any())
        if has_nan or has_pos_inf:
            raise NaNDetectedError(
                f"Non-finite values detected in attn_scores: NaN={has_nan}, Inf={has_pos_inf}",
                context={
                    "tensor_name": "attn_scores",
                    "has_nan": has_nan,
                    "has_inf": has_pos_inf,
                    "shape": list(attn_scores.shape),
                    "dtype": str(attn_scores.dtype),
                },
            )
        b, h, s_q, s_k = attn_scores.shape
        if block_size <= 0:
            raise ValueError(f"block_size must be > 0, got {block_size}")
        pad_q = (block_size - s_q % block_size) % block_size
        pad_k = (block_size - s_k % block_size) % block_size
        if pad_q > 0 or pad_k > 0:
            attn_scores = F.pad(attn_scores, (0, pad_k, 0, pad_q), value=-math.inf)
        pooled = F.max_pool2d(attn_scores, kernel_size=block_size, stride=block_size)
        nb_q, nb_k = pooled.shape[2], pooled.shape[3]
        target = F.softmax(pooled.reshape(b, h, nb_q * nb_k), dim=-1)
        return target.reshape(b, h, nb_q, nb_k)

    @staticmethod
    def compute_gate_loss(gate_soft_scores: torch.Tensor, gate_target: torch.Tensor) -> torch.Tensor:
        """KL(target || gate), "batchmean" (reference ``objectives.py:187-221``), in torch."""
        _check_finite(gate_soft_scores, "gate_soft_scores")
        _check_finite(gate_target, "gate_target")
        b, h, nb_q, nb_k = gate_soft_scores.shape
        gate_flat = gate_soft_scores.reshape(b, h, nb_q * nb_k)
        gate_dist = gate_flat / (gate_flat.sum(dim=-1, keepdim=True) + _EPS)
        target_flat = gate_target.reshape(b, h, nb_q * nb_k)
        log_gate = torch.log(gate_dist + _EPS)
        return F.kl_div(log_gate, target_flat, reduction="batchmean", log_target=False)

    @staticmethod
    def compute_sparsity_loss(gate_soft_scores: torch.Tensor, tau_target: float) -> torch.Tensor:
        """``(mean(gate_soft_scores) - tau_target) ** 2`` (reference ``objectives.py:223-240``)."""
        _check_finite(gate_soft_scores, "gate_soft_scores")
        return (gate_soft_scores.mean() - tau_target) ** 2


def gate_target_from_qk(
    q: torch.Tensor,
    k: torch.Tensor,
    block_size: int = 64,
    *,
    causal: bool = True,
    scale: float | None = None,
    normalize: str = "flat",
    temperature: float = 1.0,
    clamp: float | None = None,
    attention_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """Gate target ``[B, Hq, NB, NB]`` fp32 from ``q [B,Hq,S,D]`` and ``k [B,Hkv,S,D]`` (both
    bf16 or both fp16).

    Args:
        block_size: pooling block (32, 64 or 128).
        causal: add the ``triu(-inf, 1)`` mask of ``tasft_attention.py:434-443``.
        attention_mask: optional additive mask added to the scaled scores before the
            max-pool, as ``tasft_attention.py:445-449`` does: ``[B, S]`` is broadcast as
            ``[:, None, None, :]`` (a key-padding row), a 4-D mask must broadcast to
            ``[B, Hq, S, S]`` (e.g. HF's ``[B, 1, S, S]``). Any float or integer dtype; the
            values are added as they are. NaN or +inf raises ``NaNDetectedError`` (the
            scores would then hold them, which ``compute_gate_target`` rejects).
        scale: score scale, default ``1/sqrt(D)`` (``tasft_attention.py:427``).
        normalize: ``"flat"`` softmax over all NB*NB blocks of a head (reference trainer),
            ``"row"`` over the key blocks of each query block, ``"none"`` raw block maxima.
        temperature: divide pooled maxima by this before the softmax.
        clamp: if set, clamp finite maxima to ``[-clamp, clamp]`` first.
    """
    if q.ndim != 4 or k.ndim != 4:
        raise KernelError("Expected 4D q and k [B, H, S, D]", context={"q": list(q.shape), "k": list(k.shape)})
    B, H, S, D = q.shape
    if k.shape[0] != B or k.shape[2] != S or k.shape[3] != D or H % k.shape[1] != 0:
        raise KernelError("q and k shapes are incompatible", context={"q": list(q.shape), "k": list(k.shape)})
    if not q.is_cuda or not k.is_cuda:
        raise KernelError("Tensors must be on CUDA device", context={"device": str(q.device)})
    if k.dtype != q.dtype:
        raise KernelError("q and k must have one dtype", context={"q": str(q.dtype), "k": str(k.dtype)})
    dtype = _native.dtype_code(q.dtype, "gate target kernel")
    if normalize not in _NORMALIZE:
        raise ValueError(f"normalize must be one of {sorted(_NORMALIZE)}, got {normalize!r}")
    if not temperature > 0.0:
        raise ValueError(f"temperature must be > 0, got {temperature}")
    lib = _native.load_library()
    q = q if (q.stride(-1) == 1 and all(s % 8 == 0 for s in q.stride()[:-1])) else q.contiguous()
    k = k if (k.stride(-1) == 1 and all(s % 8 == 0 for s in k.stride()[:-1])) else k.contiguous()
    nb = math.ceil(S / block_size)
    mask_buf, mask_strides = None, None
    if attention_mask is not None:
        # The kernels read a mask up to a multiple of 64 rows and keys as well (block 32 runs
        # over 64-token blocks).
        padded = max(nb * block_size, 64 * math.ceil(S / 64))
        mask_buf, mask_strides = _padded_attention_mask(attention_mask, B, H, S, padded, q.device)
    out = torch.empty((B, H, nb, nb), dtype=torch.float32, device=q.device)
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    status = lib.tasft_gate_target_fwd(
        q.data_ptr(), k.data_ptr(), _native.ptr(mask_buf), out.data_ptr(), B, H, k.shape[1], S, D,
        block_size, _native.strides(q), _native.strides(k), mask_strides, sc, 1 if causal else 0,
        _NORMALIZE[normalize], float(temperature), float(clamp) if clamp is not None else 0.0,
        dtype, _native.stream_handle(q.device),
    )
    _native.check(status, "tasft_gate_target_fwd", {"shape": [B, H, S, D]})
    return out


def _padded_attention_mask(mask: torch.Tensor, B: int, H: int, S: int, padded: int,
                           device: torch.device):
    """The kernel's form of an additive mask: fp32 ``[B|1, H|1, padded|1, padded]`` with the
    caller's values in the leading ``S`` rows/columns (broadcast dims keep size 1 and get
    stride 0), and its (b, h, query) element strides."""
    ext = mask[:, None, None, :] if mask.ndim == 2 else mask
    if ext.ndim != 4:
        raise KernelError(f"attention_mask must be 2-D [B, S] or 4-D, got {mask.ndim}-D",
                          context={"attention_mask": list(mask.shape)})
    want = (B, H, S, S)
    if ext.shape[3] != S or any(ext.shape[i] not in (1, want[i]) for i in range(3)):
        raise KernelError(
            f"attention_mask shape {tuple(mask.shape)} does not broadcast to {want}",
            context={"attention_mask": list(mask.shape), "scores": list(want)},
        )
    ext = ext.to(device=device, dtype=torch.float32)
    has_nan = bool(torch.isnan(ext).any())
    has_pos_inf = bool((ext == float("inf")).any())
    if has_nan or has_pos_inf:
        raise NaNDetectedError(
            f"Non-finite values detected in attn_scores: NaN={has_nan}, Inf={has_pos_inf}",
            context={"tensor_name": "attention_mask", "has_nan": has_nan, "has_inf": has_pos_inf,
                     "shape": list(mask.shape), "dtype": str(mask.dtype)},
        )
    rows = padded if ext.shape[2] > 1 else 1
    buf = torch.zeros((ext.shape[0], ext.shape[1], rows, padded), dtype=torch.float32, device=device)
    buf[:, :, : ext.shape[2], :S] = ext
    st = buf.stride()
    strides = [st[0] if buf.shape[0] > 1 else 0, st[1] if buf.shape[1] > 1 else 0,
               st[2] if rows > 1 else 0]
    return buf, _native.strides_array(strides)


class _GateKL(torch.autograd.Function):
    """KL gate loss on the GPU (``tasft_gate_kl_fwd``): the loss and d(loss)/d(gate scores)
    come from one kernel; backward scales the saved gradient."""

    @staticmethod
    def forward(ctx, gate_soft: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        b, h, nbq, nbk = gate_soft.shape
        g = gate_soft.detach().to(torch.float32).contiguous()
        t = target.detach().to(torch.float32).contiguous()
        partial = torch.empty(b * h, dtype=torch.float32, device=g.device)
        grad = torch.empty_like(g) if ctx.needs_input_grad[0] else None
        lib = _native.load_library()
        status = lib.tasft_gate_kl_fwd(g.data_ptr(), t.data_ptr(), b, h, nbq, nbk, partial.data_ptr(),
                                       _native.ptr(grad), _native.stream_handle(g.device))
        _native.check(status, "tasft_gate_kl_fwd", {"shape": [b, h, nbq, nbk]})
        ctx.save_for_backward(grad)
        ctx.in_dtype = gate_soft.dtype
        return partial.sum() / b

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        (grad,) = ctx.saved_tensors
        if grad is None:
            return None, None
        return (grad * grad_out).to(ctx.in_dtype), None


def gate_loss_from_qk(
    gate_soft_scores: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    block_size: int = 64,
    *,
    causal: bool = True,
    scale: float | None = None,
    attention_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """The per-layer gate term ``compute_gate_loss(gate, compute_gate_target(scores))`` of
    ``TASFTObjective.compute`` (reference ``objectives.py:316-346``) from Q and K, without the
    ``[B, H, S, S]`` score tensor the reference's score producer stores
    (``tasft/modules/tasft_attention.py:426-458``).

    The target comes from ``gate_target_from_qk`` (MFMA block maxima, flat softmax) and
    is a constant of the loss, as the reference's detached scores are; the KL and its
    gradient with respect to ``gate_soft_scores`` come from one HIP kernel, so
    ``loss.backward()`` reaches the gate (and, through ``AttnGate``'s HIP backward, its
    parameters). NaN or Inf in ``gate_soft_scores`` raises ``NaNDetectedError``.
    """
    if gate_soft_scores.ndim != 4:
        raise KernelError("gate_soft_scores must be [B, H, NB, NB]",
                          context={"shape": list(gate_soft_scores.shape)})
    if not gate_soft_scores.is_cuda:
        raise KernelError("Tensors must be on CUDA device", context={"device": str(gate_soft_scores.device)})
    target = gate_target_from_qk(q, k, block_size, causal=causal, scale=scale,
                                 attention_mask=attention_mask)
    if tuple(target.shape) != tuple(gate_soft_scores.shape):
        raise KernelError(
            f"gate scores {tuple(gate_soft_scores.shape)} do not match the target grid {tuple(target.shape)}",
            context={"gate": list(gate_soft_scores.shape), "target": list(target.shape)})
    _check_finite(gate_soft_scores, "gate_soft_scores")
    return _GateKL.apply(gate_soft_scores, target)


__all__ = ["TASFTObjective", "gate_loss_from_qk", "gate_target_from_qk"]
