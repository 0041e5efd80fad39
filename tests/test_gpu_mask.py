"""Mask format conversions on the GPU (through the C ABI) vs the CPU oracle: exact."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import require_gpu
from oracle import tasft_oracle as orc
from tasft_amd import workloads as wl
from tasft_amd.exceptions import KernelError
from tasft_amd.kernels import BlockSparseFlashAttention, indices_to_mask, mask_to_csr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(("B", "H", "NBq", "NBk", "density", "causal"), [
    (2, 3, 7, 9, 0.3, False),
    (2, 3, 9, 9, 0.3, True),
    (1, 4, 128, 128, 0.2, True),      # config-2 row length, 2 ballots per row
    (1, 2, 3, 200, 0.05, False),      # long rows, mostly empty
    (1, 1, 5, 5, 0.0, True),          # empty mask
])
def test_mask_to_csr_matches_oracle(B, H, NBq, NBk, density, causal):
    dev = require_gpu()
    g = torch.Generator().manual_seed(NBq * 31 + NBk)
    m = torch.rand((B, H, NBq, NBk), generator=g) < density
    rp, ci = mask_to_csr(m.to(dev), causal=causal)
    rp_ref, ci_ref = orc.mask_to_csr(m.numpy(), causal)
    assert np.array_equal(rp.cpu().numpy(), rp_ref)
    assert np.array_equal(ci.cpu().numpy(), ci_ref)


def test_mask_to_csr_strided_view():
    dev = require_gpu()
    g = torch.Generator().manual_seed(9)
    big = torch.rand((2, 6, 10, 12), generator=g) < 0.4
    view = big.to(dev)[:, ::2, 1:9, 2:11]  # non-contiguous in h, rows and columns
    rp, ci = mask_to_csr(view)
    rp_ref, ci_ref = orc.mask_to_csr(big[:, ::2, 1:9, 2:11].numpy())
    assert np.array_equal(rp.cpu().numpy(), rp_ref)
    assert np.array_equal(ci.cpu().numpy(), ci_ref)


def test_indices_to_mask_matches_oracle_and_rejects_out_of_range():
    dev = require_gpu()
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(-1, 40, (4, 8, 11), generator=g, dtype=torch.int32)
    idx[0, 0] = -1          # an empty list
    idx[1, 2, :4] = 7       # duplicates
    got = indices_to_mask(idx.to(dev), 40)
    assert got.dtype == torch.bool
    assert np.array_equal(got.cpu().numpy(), orc.indices_to_mask(idx.numpy(), 40))
    bad = idx.clone()
    bad[2, 3, 5] = 40
    with pytest.raises(KernelError, match="outside"):
        indices_to_mask(bad.to(dev), 40)


def test_decode_block_indices_equal_block_mask():
    """Index-list selection gives bit-identical decode output to the equivalent mask."""
    dev = require_gpu()
    B, Hq, Hkv, S, D = 3, 8, 2, 2000, 128
    shape = wl.Shape(B, Hq, Hkv, S, D)
    nb = math.ceil(S / 64)
    q = wl.randn_bf16((B, Hq, 1, D), 41).to(dev)
    k = wl.randn_bf16((B, Hkv, S, D), 42).to(dev)
    v = wl.randn_bf16((B, Hkv, S, D), 43).to(dev)
    g = torch.Generator().manual_seed(44)
    sel = torch.stack([torch.stack([torch.randperm(nb, generator=g)[:6] for _ in range(Hq)])
                       for _ in range(B)]).to(torch.int32)  # [B, Hq, 6]
    sel[0, 1, 3:] = -1
    mask = torch.from_numpy(orc.indices_to_mask(sel.numpy(), nb)).view(B, Hq, 1, nb)
    bsfa = BlockSparseFlashAttention(block_size=64, min_sparsity_for_speedup=0.0)
    out_m = bsfa.forward_decode(q, k, v, mask.to(dev))
    out_i = bsfa.forward_decode(q, k, v, block_indices=sel.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(out_m, out_i)
    with pytest.raises(KernelError, match="exactly one"):
        bsfa.forward_decode(q, k, v, mask.to(dev), block_indices=sel.to(dev))
