"""NaN in Q, K or V: the kernels propagate it as the reference kernel does.

All device code is built with ``-fno-honor-nans``, which lets ``fmaxf`` drop a NaN
operand. The running maximum may therefore ignore a NaN score, but the NaN still reaches
the output through ``exp2`` (p and l become NaN) and through the PV product, and the
normalisation divides by ``where(l > 0, l, 1)`` (tasft/kernels/block_sparse_fa.py:255-257),
so NaN rows stay NaN instead of being turned into the empty-row 0. The expected pattern is
the block-gather oracle's, which follows the reference's per-block arithmetic: a NaN score at
an allowed element makes the row NaN; a NaN in V[j, d] reaches column d of every row whose
block row has key j's block active (0 * NaN is NaN).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import attn_inputs as ai
from helpers import assert_close_bf16, require_gpu, to_np
from oracle import tasft_oracle as orc
from tasft_amd.kernels import BlockSparseFlashAttention

pytestmark = pytest.mark.gpu

PREFILL = [
    # B, Hq, Hkv, S, D, bs (kernel: two-wave, four-wave, block 32, block 128 on block 64)
    (1, 4, 2, 700, 128, 64),
    (1, 4, 2, 700, 64, 64),
    (1, 4, 2, 300, 128, 32),
    (1, 4, 1, 700, 128, 128),
]


def _check_nan(out, ref, what):
    got = to_np(out)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref), err_msg=f"{what}: NaN pattern")
    clean = ~np.isnan(ref)
    assert np.isfinite(got[clean]).all()
    assert_close_bf16(torch.from_numpy(np.where(clean, got, 0.0)), np.where(clean, ref, 0.0), what)


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs"), PREFILL)
def test_prefill_nan_propagates_like_reference(B, Hq, Hkv, S, D, bs):
    dev = require_gpu()
    print(f"prefill NaN B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} bs={bs}", flush=True)
    q, k, v = ai.qkv("unit", (B, Hq, S, D), (B, Hkv, S, D), 9900 + S + D + bs, bs)
    q[0, 0, S // 5, 5] = float("nan")
    k[0, Hkv - 1, 2 * S // 7, 1] = float("nan")
    v[0, 0, 9 * S // 14, D - 1] = float("nan")
    nb = math.ceil(S / bs)
    mask = ai.random_mask((B, Hq, nb, nb), 0.5, 9950 + S)
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    if bs == 128:
        # Block 128 runs as its four 64-token quarters, and the quarter above the diagonal
        # is never visited: a NaN in V at a key that the causal mask hides from a row does
        # not reach it, where the reference's 128 x 128 tile multiplies it by p = 0. The
        # finite values are the same either way; the NaN pattern is that of the equivalent
        # block-64 mask.
        m64 = mask.repeat_interleave(2, -1).repeat_interleave(2, -2)[..., :math.ceil(S / 64), :math.ceil(S / 64)]
        ref = orc.attention_block_gather(qn, kn, vn, m64.numpy(), 64, True)
    else:
        ref = orc.attention_block_gather(qn, kn, vn, mask.numpy(), bs, True)
    assert np.isnan(ref).any() and not np.isnan(ref).all()
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), causal=True)
    torch.cuda.synchronize()
    _check_nan(out.cpu(), ref, f"prefill NaN D={D} bs={bs}")


def test_decode_nan_propagates():
    """Decode: a NaN key of a block selected by head h makes head h's output NaN (heads
    that do not select the block have -inf there); a NaN in V of a block that every query
    head of its KV group selects makes that column NaN for the group."""
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs = 2, 8, 2, 1000, 128, 64
    q, k, v = ai.qkv("unit", (B, Hq, 1, D), (B, Hkv, S, D), 9970, bs)
    nb = math.ceil(S / bs)
    mask = ai.random_mask((B, Hq, 1, nb), 0.4, 9971)
    mask[0, 0, 0, 3] = True        # head 0 selects block 3 ...
    mask[0, 1:4, 0, 3] = False     # ... the other heads of KV group 0 do not
    k[0, 0, 3 * 64 + 7, 11] = float("nan")
    mask[1, 4:8, 0, 9] = True      # every head of KV group 1 selects block 9
    v[1, 1, 9 * 64 + 20, 17] = float("nan")
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    ref = orc.sparse_decode(qn, kn, vn, mask.numpy(), bs)
    assert np.isnan(ref[0, 0]).all() and not np.isnan(ref[0, 1:4]).any()
    assert np.isnan(ref[1, 4:8, 0, 17]).all()
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward_decode(q.to(dev), k.to(dev), v.to(dev), mask.to(dev))
    torch.cuda.synchronize()
    _check_nan(out.cpu(), ref, "decode NaN")
