"""Cached sparse decoding for one attention layer: the gate's selection of the new token.

The reference routes decode to dense attention (``tasft/inference/vllm_patch.py:189-196``)
and its gate rejects S_q != S_k (``tasft/modules/attn_gate.py:216-221``, pinned by
``tests/integration/test_model_families.py:915-948``), so a cached decode step has no block
selection there. This module defines one: the new token at position ``t`` attends to the
key blocks its query block ``t // block`` selects in the gate row the prefill gate would
compute on the sequence ``0 .. t``, i.e. ``AttnGate.forward(q_t, k[:t+1], query_offset=t,
q_block_sum=...)``. The row's query mean is the zero-padded mean of the block's queries so
far; the key means are those of every key block so far (the last one zero-padded).

Per step nothing is pooled again: the state keeps the projected key units
``v_j = W_k kbar_j`` ([B, Hkv, blocks, hidden] fp32, from the prefill gate's workspace) and
the running sums of the current block's keys and queries, updates the one changing block,
and evaluates the row. With at most 8 query heads per KV head that is one call,
``tasft_gate_decode_rows_fwd``; otherwise torch updates the sums and projections and
``tasft_gate_rows_fwd`` evaluates the row. The row feeds
``BlockSparseFlashAttention.forward_decode`` with the KV cache in its GQA layout
(``Hkv`` heads, never repeat-interleaved as ``tasft/inference/tasft_model.py:267-271`` does).
"""
from __future__ import annotations

import math

import torch

from tasft_amd import _native
from tasft_amd.exceptions import KernelError
from tasft_amd.kernels.block_sparse_fa import (
    _VALID_HEAD_DIMS,
    BlockSparseFlashAttention,
    default_decode_splits,
)
from tasft_amd.modules.attn_gate import AttnGate, GateOutput, _launch_gate


class SparseAttentionDecoder:
    """Block-sparse prefill and cached decode steps of one layer, gate-driven.

    Args:
        gate: the layer's ``AttnGate`` (on the GPU).
        threshold: tau (float or per-head tensor ``[Hq]``); default the gate's.
        force_diagonal: keep each query block's own block (the new token's block).
        max_len: KV-cache capacity in tokens (sizes the projected key-unit state).
    """

    def __init__(self, gate: AttnGate, threshold: float | torch.Tensor | None = None, *,
                 force_diagonal: bool = True, max_len: int = 32768) -> None:
        self.gate = gate
        self.threshold = threshold if threshold is not None else gate.default_threshold
        self.force_diagonal = force_diagonal
        self.max_len = max_len
        self.bsfa = BlockSparseFlashAttention(block_size=gate.block_size, min_sparsity_for_speedup=0.0)
        self.length = 0
        self._vk = None
        self._ksum = None
        self._qsum = None
        self._ws: dict[int, tuple[torch.Tensor, int]] = {}  # decode workspace per split count
        # ctypes stride arrays per stride tuple: a step's tensors keep their strides, and
        # building the arrays was a measurable share of a step's host time.
        self._stride_arrays: dict[tuple[int, ...], object] = {}

    def _strides(self, t: torch.Tensor):
        st = t.stride()
        arr = self._stride_arrays.get(st)
        if arr is None:
            arr = _native.strides_array(st)
            self._stride_arrays[st] = arr
        return arr

    # ------------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, GateOutput]:
        """Gate + block-sparse prefill of the prompt (``q [B,Hq,S,D]``, ``k/v [B,Hkv,S,D]``
        bf16), and the decode state for the tokens that follow."""
        B, Hq, S, D = q.shape
        Hkv = k.shape[1]
        bs = self.gate.block_size
        if S > self.max_len:
            raise KernelError(f"prompt of {S} tokens exceeds max_len={self.max_len}",
                              context={"seq_len": S, "max_len": self.max_len})
        taus = self.gate._thresholds(self.threshold, q.device)
        r = _launch_gate(self.gate, q, k, taus, False, self.force_diagonal, keep=False)
        g = GateOutput(soft_scores=r["soft"], hard_mask=r["mask"].view(torch.bool), num_blocks_q=r["nb"],
                       num_blocks_k=r["nb"], active_count=r["active"])
        out = self.bsfa.forward(q, k, v, g.hard_mask, causal=self.gate.is_causal)
        hid = self.gate.gate_hidden_dim
        nb = r["nb"]
        cap = math.ceil(self.max_len / bs)
        self._vk = torch.zeros((B, Hkv, cap, hid), dtype=torch.float32, device=q.device)
        uq_bytes = B * Hq * nb * hid * 4
        uk = r["workspace"][uq_bytes:uq_bytes + B * Hkv * nb * hid * 4].view(torch.float32)
        self._vk[:, :, :nb] = uk.view(B, Hkv, nb, hid)
        last0 = (S // bs) * bs  # first token of the block the next token falls in
        if last0 < S:
            self._ksum = k[:, :, last0:S].float().sum(2)
            self._qsum = q[:, :, last0:S].float().sum(2)
        else:
            self._ksum = torch.zeros((B, Hkv, D), dtype=torch.float32, device=q.device)
            self._qsum = torch.zeros((B, Hq, D), dtype=torch.float32, device=q.device)
        self.length = S
        # Per-step constants, read from the gate once: the W_in halves with the 1/block of
        # the zero-padded mean folded in, the bias, w_out, the thresholds and the flags.
        w_in = self.gate.gate_proj_in.weight.detach().float()
        self._wk_t = (w_in[:, D:] / bs).t().contiguous()
        self._wq_t = (w_in[:, :D] / bs).t().contiguous()
        self._b_in = self.gate.gate_proj_in.bias.detach().float().contiguous()
        self._w_out = self.gate.gate_proj_out.weight.detach().float().reshape(-1).contiguous()
        self._taus = taus
        self._flags = (1 if self.gate.is_causal else 0) | (2 if self.force_diagonal else 0)
        return out, g

    # ------------------------------------------------------------------ decode
    @torch.no_grad()
    def select(self, q_new: torch.Tensor, k_new: torch.Tensor) -> GateOutput:
        """Advance the state by one token and return its gate row ``[B, Hq, 1, NB]``
        (``NB = ceil((t + 1) / block)`` for the new position ``t``)."""
        if self._vk is None:
            raise KernelError("SparseAttentionDecoder.select before prefill", context={})
        B, Hq, _, D = q_new.shape
        Hkv = k_new.shape[1]
        bs = self.gate.block_size
        t = self.length
        if t >= self.max_len:
            raise KernelError(f"KV cache full: max_len={self.max_len}", context={"length": t})
        i = t // bs
        hid = self.gate.gate_hidden_dim
        nbk = i + 1
        dev = q_new.device
        soft = torch.empty((B, Hq, 1, nbk), dtype=torch.float32, device=dev)
        mask = torch.empty((B, Hq, 1, nbk), dtype=torch.uint8, device=dev)
        active = None
        lib = _native.load_library()
        if (Hq // Hkv <= 8 and D <= 256 and hid <= 256 and hid % 4 == 0
                and q_new.dtype in (torch.bfloat16, torch.float16) and k_new.dtype == q_new.dtype
                and q_new.stride(-1) == 1 and k_new.stride(-1) == 1):
            # One launch per (b, KV head): block sums, both projections, the kept key unit of
            # block i and the rows (tasft_gate_decode_rows_fwd).
            status = lib.tasft_gate_decode_rows_fwd(
                q_new.data_ptr(), k_new.data_ptr(), self._strides(q_new), self._strides(k_new),
                self._qsum.data_ptr(), self._ksum.data_ptr(), self._vk.data_ptr(),
                self._vk.shape[2] * hid, self._wq_t.data_ptr(), self._wk_t.data_ptr(),
                self._b_in.data_ptr(), self._w_out.data_ptr(), self._taus.data_ptr(),
                # No device count: the row's sparsity is counted from the mask if asked for.
                soft.data_ptr(), mask.data_ptr(), None, B, Hq, Hkv, D, hid, i,
                1 if t % bs == 0 else 0, self._flags, _native.dtype_code(q_new.dtype, "decode rows"),
                _native.stream_handle(dev))
            _native.check(status, "tasft_gate_decode_rows_fwd", {"position": t})
        else:
            active = torch.empty((1,), dtype=torch.int64, device=dev)
            if t % bs == 0:
                self._ksum.zero_()
                self._qsum.zero_()
            self._ksum.add_(k_new[:, :, 0])
            self._qsum.add_(q_new[:, :, 0])
            self._vk[:, :, i] = torch.matmul(self._ksum, self._wk_t)
            uq = torch.addmm(self._b_in, self._qsum.view(B * Hq, D), self._wq_t).view(B, Hq, 1, hid)
            status = lib.tasft_gate_rows_fwd(
                uq.data_ptr(), self._vk.data_ptr(), self._w_out.data_ptr(), self._taus.data_ptr(),
                soft.data_ptr(), None, mask.data_ptr(), active.data_ptr(), B, Hq, Hkv, 1, nbk, i, hid,
                self._vk.shape[2] * hid, self._flags, _native.stream_handle(dev))
            _native.check(status, "tasft_gate_rows_fwd", {"position": t})
        self.length = t + 1
        return GateOutput(soft_scores=soft, hard_mask=mask.view(torch.bool), num_blocks_q=1,
                          num_blocks_k=nbk, active_count=active)

    @torch.no_grad()
    def step(self, q_new: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor
             ) -> tuple[torch.Tensor, GateOutput]:
        """One cached decode step: ``q_new [B, Hq, 1, D]``; ``k_cache``/``v_cache``
        ``[B, Hkv, t + 1, D]`` already hold the new token at position ``t`` (the HF cache
        after ``update``). Returns the attention output ``[B, Hq, 1, D]`` and the row."""
        t = self.length
        if k_cache.shape[2] != t + 1:
            raise KernelError(f"KV cache holds {k_cache.shape[2]} tokens, expected {t + 1}",
                              context={"cache_len": k_cache.shape[2], "length": t})
        row = self.select(q_new, k_cache[:, :, t:t + 1])
        return self._decode(q_new, k_cache, v_cache, row.hard_mask), row

    def _decode(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                mask: torch.Tensor) -> torch.Tensor:
        """``tasft_bsfa_decode_fwd`` on the step's row, called directly when the layouts suit
        the kernel as they are (the shapes are the decoder's own, already consistent), with
        the workspace kept between steps; ``forward_decode`` (validation, copies) otherwise."""
        B, Hq, _, D = q.shape
        Hkv, S_kv = k_cache.shape[1], k_cache.shape[2]
        ready = (D in _VALID_HEAD_DIMS and q.dtype in (torch.bfloat16, torch.float16)
                 and k_cache.dtype == q.dtype and v_cache.dtype == q.dtype and q.is_cuda
                 and all(t.stride(-1) == 1 and all(st % 8 == 0 for st in t.stride()[:-1])
                         and t.data_ptr() % 16 == 0 for t in (q, k_cache, v_cache)))
        if not ready:
            return self.bsfa.forward_decode(q, k_cache, v_cache, mask)
        lib = _native.load_library()
        nb = mask.shape[-1]
        splits = default_decode_splits(B, Hkv, nb, Hq // Hkv)
        ws = self._ws.get(splits)
        if ws is None:
            n = lib.tasft_bsfa_decode_workspace_bytes(B, Hq, D, splits)
            ws = (torch.empty(n, dtype=torch.uint8, device=q.device), n)
            self._ws[splits] = ws
        out = torch.empty((B, Hq, 1, D), dtype=q.dtype, device=q.device)
        m8 = mask.view(torch.uint8)
        status = lib.tasft_bsfa_decode_fwd(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), m8.data_ptr(),
            None, ws[0].data_ptr(), ws[1], B, Hq, Hkv, S_kv, D, self.bsfa.block_size, splits,
            self._strides(q), self._strides(k_cache), self._strides(v_cache),
            self._strides(out), self._strides(m8), 1.0 / math.sqrt(D),
            _native.dtype_code(q.dtype, "decode"), _native.stream_handle(q.device))
        _native.check(status, "tasft_bsfa_decode_fwd", {"shape": [B, Hq, S_kv, D]})
        return out


__all__ = ["SparseAttentionDecoder"]
