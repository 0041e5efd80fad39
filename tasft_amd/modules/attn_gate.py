"""AttnGate on MI355X: block mean-pool -> pairwise MLP -> sigmoid -> threshold.

Mirrors ``tasft.modules.attn_gate`` (reference ``tasft/modules/attn_gate.py:30-314``):
same constructor and defaults, the same parameters and state-dict keys
(``gate_proj_in.weight/.bias``, ``gate_proj_out.weight``) created and initialised in the
same order, the same validation order and messages, and the same ``GateOutput`` fields.

Inference on bf16 or fp16 GPU tensors (no autograd) runs the fused HIP kernels of
``libtasft_amd.so``: one pass over Q and K for the pooling (GQA-native, K pooled per KV
head) and one pairwise kernel that keeps logits, sigmoid and threshold in fp32 — gate
scores cluster within ~1e-3 of 0.5, below one bf16 ulp, so the reference's bf16 cast of
the gate would move mask bits. Those ``soft_scores`` are fp32 whatever the module dtype,
and ``sparsity_ratio`` is read from a device counter on first access instead of a sync
inside ``forward``.

Gate training on those tensors runs the same forward and a HIP backward. Everything else
the reference gate accepts — CPU tensors, fp32 Q/K, and gradients of the logits —
evaluates the reference formula itself with torch operations in the promoted dtype of the
inputs and parameters, returning ``soft_scores`` in that dtype as the reference does. It uses ``W_in . cat(x, y) = W_q x + W_k y`` (the exact
algebra of ``attn_gate.py:250-257``) so no ``[B,H,NB,NB,2D]`` tensor is built. This is the
gate's own formulation on the devices and dtypes the kernel does not serve, not a second
backend of the HIP path: a bf16 or fp16 GPU call never takes it, and fails with
``KernelError`` if the library is missing.

Additive, keyword-compatible extensions: ``k`` may have ``Hkv`` heads (``Hq % Hkv == 0``);
``threshold`` may be a per-head tensor ``[Hq]``; ``return_logits=True`` adds the logits;
``force_diagonal=True`` keeps every diagonal block.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Any

import torch
import torch.nn.functional as F
from torch import nn

from tasft_amd import _native
from tasft_amd.exceptions import KernelError, ValidationError


class GateOutput:
    """Gate result (reference ``attn_gate.py:30-46``); immutable after construction.

    Attributes:
        soft_scores: ``[B, H, NB_q, NB_k]`` scores in [0, 1] (0 above the block diagonal
            when causal): fp32 from the HIP kernel, the computation dtype otherwise.
        hard_mask: ``[B, H, NB_q, NB_k]`` bool, ``soft_scores >= threshold``.
        sparsity_ratio: fraction of False entries over the full grid (reference
            ``attn_gate.py:277``); read lazily from a device counter (or, without one, counted
            from ``hard_mask``).
        num_blocks_q, num_blocks_k: block grid size.
        logits: pre-sigmoid logits (same dtype as ``soft_scores``) when requested, else None.
    """

    __slots__ = ("soft_scores", "hard_mask", "num_blocks_q", "num_blocks_k", "logits",
                 "_sparsity", "_active", "_total")

    def __init__(
        self,
        soft_scores: torch.Tensor,
        hard_mask: torch.Tensor,
        sparsity_ratio: float | None = None,
        num_blocks_q: int = 0,
        num_blocks_k: int = 0,
        *,
        logits: torch.Tensor | None = None,
        active_count: torch.Tensor | None = None,
    ) -> None:
        # With neither, the ratio is counted from hard_mask on first access.
        init = object.__setattr__
        init(self, "soft_scores", soft_scores)
        init(self, "hard_mask", hard_mask)
        init(self, "num_blocks_q", num_blocks_q)
        init(self, "num_blocks_k", num_blocks_k)
        init(self, "logits", logits)
        init(self, "_sparsity", None if sparsity_ratio is None else float(sparsity_ratio))
        init(self, "_active", active_count)
        init(self, "_total", hard_mask.numel())

    @property
    def sparsity_ratio(self) -> float:
        if self._sparsity is None:
            if self._active is None:
                object.__setattr__(self, "_sparsity",
                                   1.0 - int(self.hard_mask.sum().item()) / max(self._total, 1))
                return self._sparsity
            active = int(self._active.item())
            if active < 0:
                # Bit 63 of the device count: the one-launch gate kernel's bounded wait for
                # its key workgroups gave up; the rows it covers hold NaN scores.
                raise KernelError(
                    "tasft_gate_fwd: a query workgroup's wait for the key units timed out; "
                    "the gate outputs of this call are invalid",
                    context={"active_count": hex(active & 0xFFFFFFFFFFFFFFFF)},
                )
            object.__setattr__(self, "_sparsity", 1.0 - active / max(self._total, 1))
        return self._sparsity

    def __setattr__(self, name: str, value: Any) -> None:
        raise dataclasses.FrozenInstanceError(f"cannot assign to field '{name}'")

    def __delattr__(self, name: str) -> None:
        raise dataclasses.FrozenInstanceError(f"cannot delete field '{name}'")

    def __repr__(self) -> str:
        return (f"GateOutput(shape={tuple(self.hard_mask.shape)}, "
                f"num_blocks_q={self.num_blocks_q}, num_blocks_k={self.num_blocks_k})")


class AttnGate(nn.Module):
    """Learnable block-importance predictor (reference ``attn_gate.py:49-311``)."""

    def __init__(
        self,
        num_heads: int,
        head_dim: int,
        block_size: int = 64,
        gate_hidden_dim: int | None = None,
        default_threshold: float = 0.5,
        is_causal: bool = True,
    ) -> None:
        super().__init__()
        if num_heads <= 0:
            raise ValidationError(f"num_heads must be positive, got {num_heads}",
                                  context={"num_heads": num_heads})
        if head_dim <= 0:
            raise ValidationError(f"head_dim must be positive, got {head_dim}",
                                  context={"head_dim": head_dim})
        if block_size <= 0:
            raise ValidationError(f"block_size must be positive, got {block_size}",
                                  context={"block_size": block_size})
        if not 0.0 <= default_threshold <= 1.0:
            raise ValidationError(f"default_threshold must be in [0, 1], got {default_threshold}",
                                  context={"default_threshold": default_threshold})
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.default_threshold = default_threshold
        self.is_causal = is_causal
        hidden = gate_hidden_dim if gate_hidden_dim is not None else max(32, head_dim // 4)
        self.gate_hidden_dim = hidden
        # Same modules in the same order as the reference, so seeded construction draws
        # the same random numbers (nn.Linear default init, then _init_weights).
        self.gate_proj_in = nn.Linear(2 * head_dim, hidden, bias=True)
        self.gate_proj_out = nn.Linear(hidden, 1, bias=False)
        self._init_weights()

    def _init_weights(self) -> None:
        """Xavier-uniform W_in, zero b_in, N(0, 0.01) W_out (reference ``attn_gate.py:140-149``)."""
        nn.init.xavier_uniform_(self.gate_proj_in.weight)
        nn.init.zeros_(self.gate_proj_in.bias)
        nn.init.normal_(self.gate_proj_out.weight, std=0.01)

    def _pool_to_blocks(self, x: torch.Tensor) -> torch.Tensor:
        """Zero-padded block mean ``[B, H, S, D] -> [B, H, NB, D]`` (reference ``:151-175``).

        Used by the differentiable training path; the inference kernel pools on device.
        """
        B, H, S, D = x.shape
        pad = (self.block_size - S % self.block_size) % self.block_size
        if pad > 0:
            x = F.pad(x, (0, 0, 0, pad))
        nb = x.shape[2] // self.block_size
        return x.view(B, H, nb, self.block_size, D).mean(dim=3)

    def _validate(self, q: torch.Tensor, k: torch.Tensor) -> None:
        """Reference checks and messages (``attn_gate.py:201-239``), GQA-aware."""
        if q.ndim != 4:
            raise ValidationError(f"Expected 4D Q tensor [B, H, S, D], got ndim={q.ndim}",
                                  context={"q_shape": list(q.shape)})
        if k.ndim != 4:
            raise ValidationError(f"Expected 4D K tensor [B, H, S, D], got ndim={k.ndim}",
                                  context={"k_shape": list(k.shape)})
        B, H, S, D = q.shape
        same = k.shape == q.shape
        gqa = (k.shape[0] == B and k.shape[2] == S and k.shape[3] == D and k.shape[1] > 0
               and H % k.shape[1] == 0)
        if not (same or gqa):
            raise ValidationError(f"Q and K must have same shape, got {q.shape} vs {k.shape}",
                                  context={"q_shape": list(q.shape), "k_shape": list(k.shape)})
        if self.num_heads != H:
            raise ValidationError(f"Expected {self.num_heads} heads, got {H}",
                                  context={"expected_heads": self.num_heads, "actual_heads": H})
        if self.head_dim != D:
            raise ValidationError(f"Expected head_dim={self.head_dim}, got {D}",
                                  context={"expected_dim": self.head_dim, "actual_dim": D})
        if S == 0:
            raise ValidationError("Sequence length must be > 0", context={"seq_len": S})

    def _needs_grad(self, q: torch.Tensor, k: torch.Tensor) -> bool:
        if not torch.is_grad_enabled():
            return False
        return q.requires_grad or k.requires_grad or any(p.requires_grad for p in self.parameters())

    def forward(
        self,
        q: torch.Tensor,
        k: torch.Tensor,
        threshold: float | torch.Tensor | None = None,
        *,
        return_logits: bool = False,
        force_diagonal: bool = False,
        query_offset: int | None = None,
        q_block_sum: torch.Tensor | None = None,
    ) -> GateOutput:
        """Block scores, hard mask and sparsity for ``q [B,H,S,D]``, ``k [B,H or Hkv,S,D]``.

        ``force_diagonal=True`` sets the diagonal blocks of ``hard_mask`` whatever their
        score (every query block then attends at least to itself).

        ``query_offset`` (keyword extension for cached decoding, where S_q != S_k; without it
        such a call raises as the reference does, ``attn_gate.py:216-221``): the queries are
        tokens ``query_offset .. query_offset + S_q - 1`` of the sequence whose keys are
        ``k``. The result holds the gate rows of the query blocks those tokens fall in,
        ``[B, H, R, ceil(S_k / block)]``, with each row's block mean taken over its tokens
        present in ``q`` plus ``q_block_sum`` (``[B, H, D]``, the sum of the queries of the
        first row's block that precede ``query_offset``; default zero), divided by the block
        size as the zero-padded pool does. For a decode step (S_q = 1, ``query_offset =
        S_k - 1``) with ``q_block_sum`` given, the row equals the last row of this gate on
        the whole sequence so far. Computed with torch operations (the serving path keeps
        the projected key blocks across steps instead: ``tasft_amd.inference``).
        """
        tau = threshold if threshold is not None else self.default_threshold
        if query_offset is not None:
            return self._forward_rows(q, k, tau, return_logits, force_diagonal, int(query_offset),
                                      q_block_sum)
        self._validate(q, k)
        if q.device != k.device:
            raise ValidationError(f"Q and K must be on the same device, got {q.device} vs {k.device}",
                                  context={"q_device": str(q.device), "k_device": str(k.device)})
        if self._kernel_applies(q, k):
            if not self._needs_grad(q, k):
                return self._forward_hip(q, k, tau, return_logits, force_diagonal)
            if not return_logits:
                return self._forward_hip_train(q, k, tau, force_diagonal)
        return self._forward_torch(q, k, tau, return_logits, force_diagonal)

    def _kernel_applies(self, q: torch.Tensor, k: torch.Tensor) -> bool:
        """The HIP kernels serve bf16 or fp16 GPU tensors (Q and K of one dtype, head_dim a
        multiple of 8, at most 256): inference, and training through the HIP backward; every
        other call (CPU, fp32 inputs, or gradients of the logits) evaluates the formula with
        torch."""
        return (q.is_cuda and q.dtype in _native.KERNEL_DTYPES and k.dtype == q.dtype
                and q.shape[-1] % 8 == 0 and q.shape[-1] <= 256)

    def _thresholds(self, tau: float | torch.Tensor, device: torch.device) -> torch.Tensor:
        if isinstance(tau, torch.Tensor):
            t = tau.to(device=device, dtype=torch.float32).reshape(-1)
            if t.numel() == 1:
                return t.expand(self.num_heads).contiguous()
            if t.numel() != self.num_heads:
                raise ValidationError(
                    f"threshold tensor must have {self.num_heads} entries, got {t.numel()}",
                    context={"threshold_shape": list(tau.shape)})
            return t.contiguous()
        return torch.full((self.num_heads,), float(tau), dtype=torch.float32, device=device)

    def _forward_hip(self, q: torch.Tensor, k: torch.Tensor, tau: float | torch.Tensor,
                     return_logits: bool, force_diagonal: bool) -> GateOutput:
        r = _launch_gate(self, q, k, self._thresholds(tau, q.device), return_logits,
                         force_diagonal, keep=False)
        return GateOutput(soft_scores=r["soft"], hard_mask=r["mask"].view(torch.bool),
                          num_blocks_q=r["nb"], num_blocks_k=r["nb"], logits=r["logits"],
                          active_count=r["active"])

    def _forward_hip_train(self, q: torch.Tensor, k: torch.Tensor, tau: float | torch.Tensor,
                           force_diagonal: bool) -> GateOutput:
        """HIP forward plus HIP backward (``tasft_gate_bwd``) through autograd: the soft
        scores carry gradients to the gate parameters (and to Q/K if they require them)
        without materialising the ``[B, H, NB, NB, hidden]`` activations."""
        taus = self._thresholds(tau, q.device)
        soft, mask, active = _HipGateFunction.apply(
            q, k, self.gate_proj_in.weight, self.gate_proj_in.bias, self.gate_proj_out.weight,
            self, taus, force_diagonal)
        nb = soft.shape[-1]
        return GateOutput(soft_scores=soft, hard_mask=mask.view(torch.bool), num_blocks_q=nb,
                          num_blocks_k=nb, logits=None, active_count=active)

    def _forward_torch(self, q: torch.Tensor, k: torch.Tensor, tau: float | torch.Tensor,
                       return_logits: bool, force_diagonal: bool) -> GateOutput:
        """The reference formula (``attn_gate.py:241-277``) with torch operations.

        Computes in the promoted dtype of Q, K and the parameters (fp32 parameters with
        bf16 inputs compute in fp32) and returns ``soft_scores`` in that dtype; the
        causal zeroing, threshold and full-grid sparsity are the reference's. Gradients
        flow to the parameters (and to Q/K if they require them).
        """
        B, H, S, D = q.shape
        Hkv = k.shape[1]
        w_in = self.gate_proj_in.weight
        dt = torch.promote_types(torch.promote_types(q.dtype, k.dtype), w_in.dtype)
        w = w_in.to(dt)
        qb = self._pool_to_blocks(q.to(dt))
        kb = self._pool_to_blocks(k.to(dt))
        if Hkv != H:
            kb = kb.repeat_interleave(H // Hkv, dim=1)
        uq = qb @ w[:, :D].t() + self.gate_proj_in.bias.to(dt)
        uk = kb @ w[:, D:].t()
        hidden = F.relu(uq.unsqueeze(3) + uk.unsqueeze(2))
        logits = (hidden @ self.gate_proj_out.weight.to(dt).t()).squeeze(-1)
        soft = torch.sigmoid(logits)
        nb = soft.shape[2]
        if self.is_causal:
            soft = soft * torch.ones(nb, nb, dtype=torch.bool, device=soft.device).tril()
        if isinstance(tau, torch.Tensor):
            hard = soft >= self._thresholds(tau, soft.device).to(dt).view(1, H, 1, 1)
        else:
            hard = soft >= tau
        if force_diagonal:
            hard = hard | torch.eye(nb, dtype=torch.bool, device=soft.device)
        active = hard.sum().reshape(1)
        return GateOutput(soft_scores=soft, hard_mask=hard, num_blocks_q=nb, num_blocks_k=nb,
                          logits=logits if return_logits else None, active_count=active)

    def _forward_rows(self, q: torch.Tensor, k: torch.Tensor, tau: float | torch.Tensor,
                      return_logits: bool, force_diagonal: bool, offset: int,
                      q_block_sum: torch.Tensor | None) -> GateOutput:
        """Gate rows for queries at ``offset ..`` against all of ``k`` (see ``forward``)."""
        if q.ndim != 4 or k.ndim != 4:
            raise ValidationError("Expected 4D Q and K tensors [B, H, S, D]",
                                  context={"q_shape": list(q.shape), "k_shape": list(k.shape)})
        B, H, Sq, D = q.shape
        Sk = k.shape[2]
        if (k.shape[0] != B or k.shape[3] != D or k.shape[1] <= 0 or H % k.shape[1] != 0
                or Sq == 0 or offset < 0 or offset + Sq > Sk):
            raise ValidationError(
                f"query_offset {offset} with Q {tuple(q.shape)} does not fit K {tuple(k.shape)}",
                context={"q_shape": list(q.shape), "k_shape": list(k.shape), "query_offset": offset})
        if self.num_heads != H:
            raise ValidationError(f"Expected {self.num_heads} heads, got {H}",
                                  context={"expected_heads": self.num_heads, "actual_heads": H})
        if self.head_dim != D:
            raise ValidationError(f"Expected head_dim={self.head_dim}, got {D}",
                                  context={"expected_dim": self.head_dim, "actual_dim": D})
        bs = self.block_size
        Hkv = k.shape[1]
        w_in = self.gate_proj_in.weight
        dt = torch.promote_types(torch.promote_types(q.dtype, k.dtype), w_in.dtype)
        r0, r1 = offset // bs, (offset + Sq - 1) // bs
        R = r1 - r0 + 1
        front = offset - r0 * bs
        qpad = F.pad(q.to(dt), (0, 0, front, R * bs - front - Sq))
        qsum = qpad.view(B, H, R, bs, D).sum(3)
        if q_block_sum is not None:
            if tuple(q_block_sum.shape) != (B, H, D):
                raise ValidationError(f"q_block_sum must have shape {(B, H, D)}, got {tuple(q_block_sum.shape)}",
                                      context={"q_block_sum": list(q_block_sum.shape)})
            qsum = qsum.clone()
            qsum[:, :, 0] += q_block_sum.to(device=qsum.device, dtype=dt)
        qb = qsum / bs
        kb = self._pool_to_blocks(k.to(dt))
        if Hkv != H:
            kb = kb.repeat_interleave(H // Hkv, dim=1)
        w = w_in.to(dt)
        uq = qb @ w[:, :D].t() + self.gate_proj_in.bias.to(dt)
        uk = kb @ w[:, D:].t()
        logits = (F.relu(uq.unsqueeze(3) + uk.unsqueeze(2)) @ self.gate_proj_out.weight.to(dt).t()).squeeze(-1)
        soft = torch.sigmoid(logits)
        nbk = soft.shape[-1]
        rows = torch.arange(r0, r1 + 1, device=soft.device)[:, None]
        cols = torch.arange(nbk, device=soft.device)[None, :]
        if self.is_causal:
            soft = soft * (cols <= rows)
        if isinstance(tau, torch.Tensor):
            hard = soft >= self._thresholds(tau, soft.device).to(dt).view(1, H, 1, 1)
        else:
            hard = soft >= tau
        if force_diagonal:
            hard = hard | (cols == rows)
        return GateOutput(soft_scores=soft, hard_mask=hard, num_blocks_q=R, num_blocks_k=nbk,
                          logits=logits if return_logits else None,
                          active_count=hard.sum().reshape(1))

    def compute_sparsity(self, soft_scores: torch.Tensor, threshold: float) -> float:
        """Fraction of scores below ``threshold`` (reference ``attn_gate.py:287-297``)."""
        return 1.0 - (soft_scores >= threshold).float().mean().item()

    @property
    def num_parameters(self) -> int:
        """Trainable parameter count (reference ``attn_gate.py:299-302``)."""
        return sum(p.numel() for p in self.parameters() if p.requires_grad)

    def extra_repr(self) -> str:
        return (
            f"num_heads={self.num_heads}, head_dim={self.head_dim}, "
            f"block_size={self.block_size}, gate_hidden_dim={self.gate_hidden_dim}, "
            f"default_threshold={self.default_threshold}, "
            f"is_causal={self.is_causal}, params={self.num_parameters}"
        )


def _kernel_layout(t: torch.Tensor) -> torch.Tensor:
    return t if (t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:-1])) else t.contiguous()


def _launch_gate(gate: AttnGate, q: torch.Tensor, k: torch.Tensor, taus: torch.Tensor,
                 return_logits: bool, force_diagonal: bool, keep: bool) -> dict:
    """Run ``tasft_gate_fwd``; with ``keep`` also return the block means and the workspace
    (the projected units) that the backward needs."""
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    lib = _native.load_library()
    dev = q.device
    q = _kernel_layout(q.detach())
    k = _kernel_layout(k.detach())
    w_in = gate.gate_proj_in.weight.detach().to(device=dev, dtype=torch.float32).contiguous()
    b_in = gate.gate_proj_in.bias.detach().to(device=dev, dtype=torch.float32).contiguous()
    w_out = gate.gate_proj_out.weight.detach().to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    nb = math.ceil(S / gate.block_size)
    hidden = gate.gate_hidden_dim
    soft = torch.empty((B, H, nb, nb), dtype=torch.float32, device=dev)
    mask = torch.empty((B, H, nb, nb), dtype=torch.uint8, device=dev)
    logits = torch.empty((B, H, nb, nb), dtype=torch.float32, device=dev) if return_logits else None
    active = torch.empty((1,), dtype=torch.int64, device=dev)
    qm = torch.empty((B, H, nb, D), dtype=torch.float32, device=dev) if keep else None
    km = torch.empty((B, Hkv, nb, D), dtype=torch.float32, device=dev) if keep else None
    ws_bytes = lib.tasft_gate_workspace_bytes(B, H, Hkv, S, D, gate.block_size, hidden)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    status = lib.tasft_gate_fwd(
        q.data_ptr(), k.data_ptr(), w_in.data_ptr(), b_in.data_ptr(), w_out.data_ptr(),
        taus.data_ptr(), soft.data_ptr(), _native.ptr(logits), mask.data_ptr(), active.data_ptr(),
        _native.ptr(qm), _native.ptr(km), workspace.data_ptr(), ws_bytes, B, H, Hkv, S, D,
        gate.block_size, hidden, _native.strides(q), _native.strides(k),
        (1 if gate.is_causal else 0) | (2 if force_diagonal else 0),
        _native.dtype_code(q.dtype, "tasft_gate_fwd"), _native.stream_handle(dev),
    )
    _native.check(status, "tasft_gate_fwd", {"shape": [B, H, S, D]})
    return {"soft": soft, "mask": mask, "logits": logits, "active": active, "nb": nb,
            "q_means": qm, "k_means": km, "workspace": workspace, "w_in": w_in, "w_out": w_out}


def _weight_grad(d: torch.Tensor, m: torch.Tensor, chunk: int = 256) -> torch.Tensor:
    """``d^T @ m`` for tall fp32 operands ([K, hidden] and [K, D], K = B * H * NB).

    The output is one small tile while K runs to tens of thousands, so a single GEMM runs
    on a handful of workgroups that each walk all of K. Split K into chunks of ``chunk``
    rows as a batched product and sum the partial products instead (K not a multiple of
    ``chunk``, or a single chunk: one plain GEMM).
    """
    K = d.shape[0]
    if K % chunk or K < 2 * chunk:
        return d.t() @ m
    c = K // chunk
    return torch.bmm(d.view(c, chunk, -1).transpose(1, 2), m.view(c, chunk, -1)).sum(0)


class _HipGateFunction(torch.autograd.Function):
    """AttnGate forward/backward on the HIP kernels (gate training).

    Backward, with g = dL/dsoft * soft * (1 - soft) (0 where the causal zero applied) and
    pre_ijc = u_ic + v_jc (u = W_q qbar + b_in, v = W_k kbar): ``tasft_gate_bwd`` reduces
    the pairwise terms; the rest are plain GEMMs on [B, H, NB, .] tensors:
      dL/dw_out = sum g relu(pre);  dL/du = w_out * sum_j g [pre > 0];
      dL/dv = w_out * sum_i g [pre > 0] (summed over the query heads of each KV head);
      dL/db_in = sum du;  dL/dW_in = [du^T qbar, dv^T kbar];
      dL/dqbar = du W_q, dL/dkbar = dv W_k, spread over each block's tokens / block size.
    """

    @staticmethod
    def forward(ctx, q, k, w_in, b_in, w_out, gate, taus, force_diagonal):
        r = _launch_gate(gate, q, k, taus, False, force_diagonal, keep=True)
        ctx.gate_cfg = (gate.block_size, gate.gate_hidden_dim, gate.is_causal)
        ctx.shapes = (tuple(q.shape), tuple(k.shape))
        ctx.dtypes = (q.dtype, k.dtype, w_in.dtype, b_in.dtype, w_out.dtype)
        ctx.save_for_backward(r["soft"], r["workspace"], r["q_means"], r["k_means"], r["w_in"],
                              r["w_out"])
        ctx.mark_non_differentiable(r["mask"], r["active"])
        return r["soft"], r["mask"], r["active"]

    @staticmethod
    def backward(ctx, grad_soft, _grad_mask, _grad_active):
        soft, workspace, qm, km, w_in, w_out = ctx.saved_tensors
        bs, hidden, causal = ctx.gate_cfg
        (B, H, S, D), (_, Hkv, _, _) = ctx.shapes
        nb = soft.shape[-1]
        lib = _native.load_library()
        dev = soft.device
        gs = grad_soft.to(torch.float32).contiguous()
        pbytes = lib.tasft_gate_bwd_workspace_bytes(B, H, S, bs, hidden)
        partials = torch.empty(pbytes // 4, dtype=torch.float32, device=dev)
        status = lib.tasft_gate_bwd(soft.data_ptr(), gs.data_ptr(), workspace.data_ptr(),
                                    workspace.numel(), partials.data_ptr(), pbytes, B, H, Hkv, S,
                                    bs, hidden, 1 if causal else 0, _native.stream_handle(dev))
        _native.check(status, "tasft_gate_bwd", {"shape": [B, H, S, D]})
        tiles = (nb + 31) // 32
        plane = B * H * nb * hidden
        du = partials[: tiles * plane].view(tiles, B, H, nb, hidden).sum(0) * w_out
        dv = (partials[tiles * plane: 2 * tiles * plane].view(tiles, B, Hkv, H // Hkv, nb, hidden)
              .sum((0, 3)) * w_out)
        dw_out = partials[2 * tiles * plane:].view(-1, hidden).sum(0)
        db_in = du.sum((0, 1, 2))
        dw_q = _weight_grad(du.reshape(-1, hidden), qm.reshape(-1, D))
        dw_k = _weight_grad(dv.reshape(-1, hidden), km.reshape(-1, D))
        dw_in = torch.cat([dw_q, dw_k], dim=1)
        gq = gk = None
        if ctx.needs_input_grad[0]:
            dqbar = (du @ w_in[:, :D]) / bs
            gq = dqbar.repeat_interleave(bs, dim=2)[:, :, :S].to(ctx.dtypes[0])
        if ctx.needs_input_grad[1]:
            dkbar = (dv @ w_in[:, D:]) / bs
            gk = dkbar.repeat_interleave(bs, dim=2)[:, :, :S].to(ctx.dtypes[1])
        return (gq, gk, dw_in.to(ctx.dtypes[2]), db_in.to(ctx.dtypes[3]),
                dw_out.view(1, -1).to(ctx.dtypes[4]), None, None, None)


__all__ = ["AttnGate", "GateOutput"]
