"""Attention test inputs whose softmax is far from uniform, and the cases that use them.

At the benchmark scale (Q, K ~ N(0,1)/sqrt(128)) the scaled scores have a standard
deviation of about 0.008, so the softmax is within about 1% of uniform and a kernel with
a wrong QK^T, a wrong exp2 scale or broken max tracking still meets the parity bar. The
kinds below make those mistakes visible:

* ``base``: N(0,1)/sqrt(128) for Q, K and V (the benchmark distribution);
* ``unit``: N(0,1) for Q, K and V, so std(QK^T * scale) is about 1;
* ``peaky``: ``unit`` with key block j of every sequence multiplied by
  ``min(1 + 0.5 j, 6)``, doubled again when ``j % 4 == 3``. Scores grow along the key
  axis, with jumps of more than 8 log2 units from one block to the next, so every kernel's
  running maximum has to move (its lazy rescale fires), several times per row.

``tests/test_discriminating_inputs.py`` checks on the CPU that on every case listed here an
oracle with uniform weights (scale 0) or with twice the scale fails the parity bar, while a
bf16 emulation of the kernel arithmetic passes it.
"""
from __future__ import annotations

import math

import numpy as np
import torch

KINDS = ("base", "unit", "peaky")


def key_block_factor(pos: np.ndarray | torch.Tensor, bs: int) -> torch.Tensor:
    """Multiplier of the ``peaky`` kind for keys at positions ``pos`` (within a sequence)."""
    j = torch.as_tensor(pos) // bs
    f = torch.clamp(1.0 + 0.5 * j.float(), max=6.0)
    return torch.where(j % 4 == 3, 2.0 * f, f)


def _randn(shape, g, kind):
    x = torch.randn(shape, generator=g, dtype=torch.float32)
    return x / math.sqrt(128) if kind == "base" else x


def qkv(kind: str, q_shape, kv_shape, seed: int, bs: int, seq_axis: int = 2,
        dtype: torch.dtype = torch.bfloat16):
    """CPU tensors q, k, v of ``dtype``; ``seq_axis`` is the token axis of K (for ``peaky``)."""
    if kind not in KINDS:
        raise ValueError(kind)
    g = torch.Generator().manual_seed(seed)
    q = _randn(q_shape, g, kind)
    k = _randn(kv_shape, g, kind)
    v = _randn(kv_shape, g, kind)
    if kind == "peaky":
        n = kv_shape[seq_axis]
        f = key_block_factor(torch.arange(n), bs)
        view = [1] * len(kv_shape)
        view[seq_axis] = n
        k = k * f.view(view)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def packed_qkv(kind: str, lens: list[int], hq: int, hkv: int, d: int, seed: int, bs: int,
               pad: int = 5, dtype: torch.dtype = torch.bfloat16):
    """Packed ``q [T, Hq, D]``, ``k/v [T, Hkv, D]`` (T = sum(lens) + pad) and cu_seqlens.

    For ``peaky`` the key factor follows each token's position within its own sequence.
    """
    g = torch.Generator().manual_seed(seed)
    t = sum(lens) + pad
    q = _randn((t, hq, d), g, kind)
    k = _randn((t, hkv, d), g, kind)
    v = _randn((t, hkv, d), g, kind)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    if kind == "peaky":
        pos = torch.zeros(t, dtype=torch.int64)
        for n0, n1 in zip(cu[:-1], cu[1:]):
            pos[n0:n1] = torch.arange(n1 - n0)
        k = k * key_block_factor(pos, bs).view(t, 1, 1)
    return q.to(dtype), k.to(dtype), v.to(dtype), cu


def random_mask(shape, density: float, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.rand(shape, generator=g) < density


# ----------------------------------------------------------------------------- cases
# Prefill: (B, Hq, Hkv, S, D, bs, causal, density, variant). ``variant`` names the kernel
# the shape selects: "2w" the two-wave block-64 D=128 kernel; "4w" the four-wave block-64
# D=64 kernel (run both with and without its persistent work queue); "gen" the generic
# kernel (block 32 or 128).
PREFILL_CASES = [
    (1, 8, 2, 1000, 128, 64, True, 0.45, "2w"),
    (2, 4, 4, 384, 128, 64, False, 0.5, "2w"),
    (1, 4, 2, 700, 64, 64, True, 0.5, "4w"),
    (1, 4, 1, 448, 64, 64, False, 0.5, "4w"),
    (1, 4, 2, 600, 128, 32, True, 0.4, "gen"),
    (1, 2, 2, 520, 64, 128, True, 0.6, "gen"),
    (1, 4, 4, 300, 64, 32, False, 0.5, "gen"),
    # Rows longer than 128 key blocks (three 64-byte mask chunks per row), G=7.
    (1, 7, 1, 8300, 128, 64, True, 0.08, "2w"),
    (1, 2, 1, 8300, 128, 64, False, 0.08, "2w"),
]

# Varlen prefill: (lens, Hq, Hkv, D, bs, causal, density).
VARLEN_CASES = [
    ([300, 0, 257, 64, 1], 8, 2, 128, 64, True, 0.5),
    ([300, 45, 200], 4, 4, 64, 64, True, 0.5),
    ([330, 77], 4, 2, 64, 32, False, 0.6),
    ([513, 200], 7, 1, 128, 128, True, 0.5),
]

# Contiguous decode: (B, Hq, Hkv, S_kv, D, bs, density, splits); splits None = default.
DECODE_CASES = [
    (2, 8, 2, 1500, 128, 64, 0.4, 1),
    (2, 8, 2, 1500, 128, 64, 0.4, 3),
    (3, 8, 2, 1000, 128, 64, 0.3, None),
    (2, 7, 1, 777, 128, 64, 0.4, 2),
    (1, 8, 8, 600, 64, 32, 0.5, None),
    (2, 8, 2, 1024, 128, 128, 0.5, None),
    (2, 32, 2, 1200, 128, 64, 0.4, 2),      # 16 query heads per KV head
]

# Paged decode: (B, Hq, Hkv, S, D, bs, page_size, splits).
PAGED_CASES = [
    (3, 32, 8, 1000, 128, 64, 16, None),
    (2, 8, 2, 900, 128, 64, 64, 1),
    (2, 8, 1, 700, 64, 32, 16, 3),
    (2, 8, 2, 1000, 128, 128, 16, None),
    (2, 32, 2, 900, 128, 64, 16, None),     # 16 query heads per KV head
]


# fp16 runs of the same kernels: one case per prefill kernel variant and block size, and
# decode with one and several splits, with GQA and without.
F16_PREFILL_CASES = [PREFILL_CASES[i] for i in (0, 2, 3, 4, 5)]
F16_DECODE_CASES = [DECODE_CASES[i] for i in (0, 1, 4, 5)]


def prefill_case_inputs(case, kind: str, dtype: torch.dtype = torch.bfloat16):
    """Inputs of one prefill case: ``q, k, v, mask`` (CPU)."""
    B, Hq, Hkv, S, D, bs, causal, density, _variant = case
    seed = 9100 + S + 7 * Hq + D + bs + KINDS.index(kind)
    q, k, v = qkv(kind, (B, Hq, S, D), (B, Hkv, S, D), seed, bs, dtype=dtype)
    nb = math.ceil(S / bs)
    mask = random_mask((B, Hq, nb, nb), density, seed + 1)
    return q, k, v, mask


def varlen_case_inputs(case, kind: str, dtype: torch.dtype = torch.bfloat16):
    """Inputs of one varlen case: ``q, k, v, cu, mask`` (CPU)."""
    lens, Hq, Hkv, D, bs, causal, density = case
    seed = 9300 + sum(lens) + D + bs + KINDS.index(kind)
    q, k, v, cu = packed_qkv(kind, lens, Hq, Hkv, D, seed, bs, dtype=dtype)
    nb = math.ceil(max(lens) / bs)
    mask = random_mask((len(lens), Hq, nb, nb), density, seed + 1)
    return q, k, v, cu, mask


def decode_case_inputs(case, kind: str, dtype: torch.dtype = torch.bfloat16):
    """Inputs of one decode case: ``q, k_cache, v_cache, mask`` (CPU); head (0, 0) selects
    nothing (its output must be exactly 0)."""
    B, Hq, Hkv, S, D, bs, density, _splits = case
    seed = 9500 + S + Hq + D + bs + KINDS.index(kind)
    q, k, v = qkv(kind, (B, Hq, 1, D), (B, Hkv, S, D), seed, bs, dtype=dtype)
    nb = math.ceil(S / bs)
    mask = random_mask((B, Hq, 1, nb), density, seed + 1)
    mask[0, 0] = False
    return q, k, v, mask


def paged_case_inputs(case, kind: str, dtype: torch.dtype = torch.bfloat16):
    """Inputs of one paged-decode case.

    Returns ``q, k, v`` (contiguous caches ``[B, Hkv, cap, D]``), ``k_pages, v_pages``
    (``[n_pages, page_size, Hkv, D]``), ``table [B, per]`` int32, ``lens [B]`` int32 and
    ``mask [B, Hq, 1, NB]``. The pages of every sequence sit in a random order among spare
    pages of noise; ``lens[0]`` is the full length.
    """
    B, Hq, Hkv, S, D, bs, ps, _splits = case
    seed = 9700 + S + ps + D + KINDS.index(kind)
    per = (S + ps - 1) // ps
    cap = per * ps
    q, k, v = qkv(kind, (B, Hq, 1, D), (B, Hkv, cap, D), seed, bs, dtype=dtype)
    g = torch.Generator().manual_seed(seed + 1)
    lens = torch.randint(1, S + 1, (B,), generator=g, dtype=torch.int32)
    lens[0] = S
    nb = (cap + bs - 1) // bs
    mask = torch.rand((B, Hq, 1, nb), generator=g) < 0.4
    mask[:, :, :, 0] = True
    n_pages = B * per + 7
    perm = torch.randperm(n_pages, generator=g)
    table = perm[: B * per].view(B, per).to(torch.int32)
    kp = torch.randn(n_pages, ps, Hkv, D, generator=g).to(dtype)
    vp = torch.randn(n_pages, ps, Hkv, D, generator=g).to(dtype)
    for b in range(B):
        for j in range(per):
            kp[table[b, j]] = k[b, :, j * ps:(j + 1) * ps].transpose(0, 1)
            vp[table[b, j]] = v[b, :, j * ps:(j + 1) * ps].transpose(0, 1)
    return q, k, v, kp, vp, table, lens, mask


def case_id(case) -> str:
    return "-".join(str(x).replace(" ", "") for x in case)
