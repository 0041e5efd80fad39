"""Split-K decode parity: HIP vs the CPU oracle, and vs the prefill kernel's last row."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import attn_inputs as ai
from helpers import assert_close_bf16, require_gpu, to_np
from oracle import tasft_oracle as orc
from tasft_amd import workloads as wl
from tasft_amd.kernels import BlockSparseFlashAttention, default_decode_splits

pytestmark = pytest.mark.gpu


def _decode(q, kc, vc, mask, bs, kv_lens=None, num_splits=None):
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward_decode(q, kc, vc, mask, kv_lens=kv_lens, num_splits=num_splits)
    torch.cuda.synchronize()
    return out


CASES = [
    # B, Hq, Hkv, S_kv, D, bs, density, splits
    (3, 8, 2, 1000, 128, 64, 0.3, None),
    (2, 4, 4, 640, 128, 64, 0.5, 1),        # MHA, single split
    (2, 7, 1, 777, 128, 64, 0.25, 3),       # G=7, ragged, odd split count
    (1, 8, 8, 300, 64, 32, 0.4, 64),        # D=64, bs=32, more splits than blocks
    (2, 8, 2, 1024, 128, 128, 0.5, None),   # bs=128
    (4, 32, 8, 4096, 128, 64, 0.1, None),   # config-3 grouping at a smaller cache
    (1, 8, 2, 40000, 128, 64, 0.05, 1),     # 625 blocks in one split (no combine pass)
    (2, 8, 2, 20000, 128, 64, 0.2, 2),      # splits share the selected blocks of a row
    (2, 32, 2, 1500, 128, 64, 0.3, None),   # 16 query heads per KV head (every MFMA column)
    (2, 24, 2, 900, 64, 32, 0.4, 3),        # 12 heads, D=64, bs=32, combine pass
    (1, 16, 1, 1300, 128, 128, 0.4, 1),     # 16 heads at block 128
]


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs", "density", "splits"), CASES)
def test_decode_matches_oracle(B, Hq, Hkv, S, D, bs, density, splits):
    dev = require_gpu()
    seed = 100 + S
    q = wl.randn_bf16((B, Hq, 1, D), seed)
    kc = wl.randn_bf16((B, Hkv, S, D), seed + 1)
    vc = wl.randn_bf16((B, Hkv, S, D), seed + 2)
    nb = math.ceil(S / bs)
    g = torch.Generator().manual_seed(seed)
    mask = torch.rand((B, Hq, 1, nb), generator=g) < density  # independent per query head
    mask[0, 0] = False  # a head with nothing selected -> exact 0
    out = _decode(q.to(dev), kc.to(dev), vc.to(dev), mask.to(dev), bs, num_splits=splits)
    assert (out[0, 0].cpu() == 0).all()
    ref = orc.sparse_decode(to_np(q), to_np(kc), to_np(vc), mask.numpy(), bs)
    assert_close_bf16(out, ref, f"decode {B}x{Hq}/{Hkv}x{S} bs={bs} splits={splits}")


@pytest.mark.parametrize("kind", ("unit", "peaky"))
@pytest.mark.parametrize("case", ai.DECODE_CASES, ids=ai.case_id)
def test_decode_discriminating_inputs(case, kind):
    """Scores far from uniform: pins QK^T, the exp2 scale, per-wave max tracking, the lazy
    rescale and the merge of waves and splits (one split with direct writes, and several
    with the combine kernel)."""
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs, _dens, splits = case
    print(f"decode discriminating {case} {kind}", flush=True)
    q, kc, vc, mask = ai.decode_case_inputs(case, kind)
    out = _decode(q.to(dev), kc.to(dev), vc.to(dev), mask.to(dev), bs, num_splits=splits)
    assert (out[0, 0].cpu() == 0).all()
    ref = orc.sparse_decode(to_np(q), to_np(kc), to_np(vc), mask.numpy(), bs)
    assert_close_bf16(out, ref, f"decode {case} {kind}")
    lens = torch.randint(1, S + 1, (B,), generator=torch.Generator().manual_seed(S))
    out = _decode(q.to(dev), kc.to(dev), vc.to(dev), mask.to(dev), bs,
                  kv_lens=lens.to(torch.int32).to(dev), num_splits=splits)
    ref = orc.sparse_decode(to_np(q), to_np(kc), to_np(vc), mask.numpy(), bs, kv_lens=lens.numpy())
    assert_close_bf16(out, ref, f"decode {case} {kind} kv_lens")


def test_decode_kv_lens():
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs = 4, 8, 2, 700, 128, 64
    q = wl.randn_bf16((B, Hq, 1, D), 7)
    kc = wl.randn_bf16((B, Hkv, S, D), 8)
    vc = wl.randn_bf16((B, Hkv, S, D), 9)
    nb = math.ceil(S / bs)
    mask = torch.rand((B, Hq, 1, nb), generator=torch.Generator().manual_seed(7)) < 0.6
    lens = torch.tensor([700, 1, 64, 333], dtype=torch.int32)
    out = _decode(q.to(dev), kc.to(dev), vc.to(dev), mask.to(dev), bs, kv_lens=lens.to(dev))
    ref = orc.sparse_decode(to_np(q), to_np(kc), to_np(vc), mask.numpy(), bs, kv_lens=lens.numpy())
    assert_close_bf16(out, ref, "decode kv_lens")


def test_decode_equals_prefill_last_row():
    """The decode of token S-1 equals row S-1 of the prefill under the same mask row."""
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs = 2, 8, 2, 960, 128, 64
    q, k, v = wl.qkv(wl.Shape(B, Hq, Hkv, S, D), 55)
    nb = S // bs
    row = torch.rand((B, Hq, 1, nb), generator=torch.Generator().manual_seed(55)) < 0.4
    row[..., nb - 1] = True
    full = torch.zeros((B, Hq, nb, nb), dtype=torch.bool)
    full[:, :, nb - 1, :] = row[:, :, 0, :]
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    pre = bsfa.forward(qd, kd, vd, full.to(dev), causal=True)
    dec = bsfa.forward_decode(qd[:, :, S - 1 : S].contiguous(), kd, vd, row.to(dev))
    torch.cuda.synchronize()
    diff = (pre[:, :, S - 1].float() - dec[:, :, 0].float()).abs()
    assert float(diff.max()) <= 1e-2, f"decode vs prefill last row: {float(diff.max())}"


def test_config3_full_size_default_splits():
    """Config 3 as benchmarked: B=64, S_kv=32768, 32/8 heads, 51 of 512 blocks per KV head
    (sink and recent kept), the default split count (one split per (b, KV head), direct
    writes, 512 workgroups). K/V are drawn on the device as the bench does; sampled
    (b, h) pairs are compared with the oracle on slices copied back. The same launch runs
    again on unit-scale Q/K/V."""
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[3]
    bsfa = BlockSparseFlashAttention(block_size=shape.block, min_sparsity_for_speedup=0.0)
    nb = shape.nb
    assert default_decode_splits(shape.batch, shape.kv_heads, nb) == 1
    grp = shape.q_heads // shape.kv_heads
    gen = torch.Generator(device=dev).manual_seed(1003)
    kv_shape = (shape.batch, shape.kv_heads, shape.seq, shape.head_dim)
    kc = torch.randn(kv_shape, generator=gen, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(kv_shape, generator=gen, device=dev, dtype=torch.bfloat16)
    mask = wl.decode_mask(shape, 51, 2003)
    assert int(mask[0, 0, 0].sum()) == 51 and bool(mask[0, 0, 0, 0]) and bool(mask[0, 0, 0, -1])
    md = mask.to(dev)
    pairs = [(0, 0), (17, 9), (40, 22), (63, 31)]
    for kind in ("base", "unit"):
        print(f"config 3 B=64 {kind}", flush=True)
        if kind == "base":
            q = wl.randn_bf16((shape.batch, shape.q_heads, 1, shape.head_dim), 1003)
            kd = kc * (1.0 / math.sqrt(shape.head_dim))
            vd = vc * (1.0 / math.sqrt(shape.head_dim))
        else:
            q = wl.randn_bf16((shape.batch, shape.q_heads, 1, shape.head_dim), 1013, scale=1.0)
            kd, vd = kc, vc
        out = _decode(q.to(dev), kd, vd, md, shape.block).cpu()
        assert torch.isfinite(out.float()).all()
        for b, h in pairs:
            kvh = h // grp
            ref = orc.sparse_decode(to_np(q[b:b + 1, h:h + 1]), to_np(kd[b:b + 1, kvh:kvh + 1]),
                                    to_np(vd[b:b + 1, kvh:kvh + 1]), mask[b:b + 1, h:h + 1].numpy(),
                                    shape.block)
            assert_close_bf16(out[b:b + 1, h:h + 1], ref, f"config 3 {kind} ({b},{h})")
        del kd, vd


def test_qwen_geometry_full_size_default_splits():
    """Seven query heads per KV head (Qwen-2.5-7B: 28/4 heads; seven of the kernel's 16 MFMA
    head columns carry a query), at the config-3 batch and cache (B=64, S_kv=32768,
    51 of 512 blocks per KV head): the default is one split per (b, KV head), 256
    workgroups, direct writes. Unit-scale Q/K/V drawn on the device; sampled (b, h) pairs,
    including the last head of a group, against the oracle."""
    dev = require_gpu()
    shape = wl.Shape(64, 28, 4, 32768)
    nb = shape.nb
    assert default_decode_splits(shape.batch, shape.kv_heads, nb, 7) == 1
    gen = torch.Generator(device=dev).manual_seed(1023)
    kv_shape = (shape.batch, shape.kv_heads, shape.seq, shape.head_dim)
    kc = torch.randn(kv_shape, generator=gen, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(kv_shape, generator=gen, device=dev, dtype=torch.bfloat16)
    mask = wl.decode_mask(shape, 51, 2023)
    q = wl.randn_bf16((shape.batch, shape.q_heads, 1, shape.head_dim), 1033, scale=1.0)
    print("qwen decode geometry B=64 28/4", flush=True)
    out = _decode(q.to(dev), kc, vc, mask.to(dev), shape.block).cpu()
    assert torch.isfinite(out.float()).all()
    for b, h in [(0, 0), (9, 6), (33, 13), (63, 27)]:
        kvh = h // 7
        ref = orc.sparse_decode(to_np(q[b:b + 1, h:h + 1]), to_np(kc[b:b + 1, kvh:kvh + 1]),
                                to_np(vc[b:b + 1, kvh:kvh + 1]), mask[b:b + 1, h:h + 1].numpy(),
                                shape.block)
        assert_close_bf16(out[b:b + 1, h:h + 1], ref, f"qwen decode ({b},{h})")


# ----------------------------------------------------------------------------- paged cache
PAGED_CASES = [
    # B, Hq, Hkv, S, D, bs, page_size, splits
    (3, 32, 8, 1000, 128, 64, 16, None),   # vLLM's default page size, partial last block
    (2, 8, 2, 777, 128, 64, 32, 1),        # one split: direct write, no combine
    (2, 4, 4, 512, 64, 64, 64, None),      # page = block, D=64
    (2, 8, 1, 300, 128, 32, 64, None),     # page larger than the block
    (1, 16, 2, 640, 64, 32, 16, 3),
    (3, 32, 8, 1000, 128, 128, 16, None),  # block 128 (two 64-key halves), partial last block
    (2, 8, 2, 900, 64, 128, 64, 2),
    (2, 8, 2, 700, 128, 64, 8, None),      # 8-token pages: a 16-key tile spans two pages
    (1, 4, 1, 333, 64, 32, 8, 2),
]


def _contig_reference(bsfa, q, k, v, mask, lens, splits):
    """The contiguous decode the paged one must equal bit for bit. A block-128 mask runs on
    the 64-key kernel, as the contiguous call on the same mask expanded to 64-key blocks."""
    if bsfa.block_size != 128:
        return bsfa.forward_decode(q, k, v, mask, kv_lens=lens, num_splits=splits)
    nb64 = math.ceil(k.shape[2] / 64)
    m64 = mask.repeat_interleave(2, -1)[..., :nb64].contiguous()
    return BlockSparseFlashAttention(block_size=64, min_sparsity_for_speedup=0.0).forward_decode(
        q, k, v, m64, kv_lens=lens, num_splits=splits)


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs", "ps", "splits"), PAGED_CASES)
def test_decode_paged_equals_contiguous_and_oracle(B, Hq, Hkv, S, D, bs, ps, splits):
    dev = require_gpu()
    print(f"paged decode B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} bs={bs} ps={ps}", flush=True)
    g = torch.Generator().manual_seed(7000 + S + ps)
    per = (S + ps - 1) // ps
    cap = per * ps
    q = (torch.randn(B, Hq, 1, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    k = (torch.randn(B, Hkv, cap, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    v = (torch.randn(B, Hkv, cap, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    lens = torch.randint(1, S + 1, (B,), generator=g, dtype=torch.int32)
    lens[0] = S
    nb = (cap + bs - 1) // bs
    mask = torch.rand((B, Hq, 1, nb), generator=g) < 0.4
    mask[:, :, :, 0] = True
    # Pools: the pages of every sequence in a random order among spare pages of noise.
    n_pages = B * per + 7
    perm = torch.randperm(n_pages, generator=g)
    table = perm[: B * per].view(B, per).to(torch.int32)
    kp = torch.randn(n_pages, ps, Hkv, D, generator=g).to(torch.bfloat16)
    vp = torch.randn(n_pages, ps, Hkv, D, generator=g).to(torch.bfloat16)
    for b in range(B):
        for j in range(per):
            kp[table[b, j]] = k[b, :, j * ps:(j + 1) * ps].transpose(0, 1)
            vp[table[b, j]] = v[b, :, j * ps:(j + 1) * ps].transpose(0, 1)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    paged = bsfa.forward_decode_paged(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev),
                                      lens.to(dev), mask.to(dev), num_splits=splits)
    contig = _contig_reference(bsfa, q.to(dev), k.to(dev), v.to(dev), mask.to(dev), lens.to(dev), splits)
    torch.cuda.synchronize()
    assert torch.equal(paged, contig)
    ref = orc.sparse_decode_paged(to_np(q), to_np(kp), to_np(vp), table.numpy(), lens.numpy(),
                                  mask.numpy(), bs)
    assert_close_bf16(paged, ref, f"paged decode ps={ps}")


@pytest.mark.parametrize("kind", ("unit", "peaky"))
@pytest.mark.parametrize("case", ai.PAGED_CASES, ids=ai.case_id)
def test_decode_paged_discriminating_inputs(case, kind):
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs, ps, splits = case
    print(f"paged decode discriminating {case} {kind}", flush=True)
    q, k, v, kp, vp, table, lens, mask = ai.paged_case_inputs(case, kind)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    paged = bsfa.forward_decode_paged(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev),
                                      lens.to(dev), mask.to(dev), num_splits=splits)
    contig = _contig_reference(bsfa, q.to(dev), k.to(dev), v.to(dev), mask.to(dev), lens.to(dev), splits)
    torch.cuda.synchronize()
    assert torch.equal(paged, contig)
    ref = orc.sparse_decode_paged(to_np(q), to_np(kp), to_np(vp), table.numpy(), lens.numpy(),
                                  mask.numpy(), bs)
    assert_close_bf16(paged, ref, f"paged decode {case} {kind}")


def test_decode_paged_block_indices_equals_mask():
    """Index-list selection on a paged cache equals the dense-mask call."""
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs, ps = 2, 8, 2, 512, 128, 64, 16
    g = torch.Generator().manual_seed(7300)
    per = S // ps
    q = (torch.randn(B, Hq, 1, D, generator=g) / math.sqrt(D)).to(torch.bfloat16).to(dev)
    kp = (torch.randn(B * per, ps, Hkv, D, generator=g) / math.sqrt(D)).to(torch.bfloat16).to(dev)
    vp = torch.randn(B * per, ps, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    table = torch.randperm(B * per, generator=g).view(B, per).to(torch.int32).to(dev)
    lens = torch.tensor([S, 300], dtype=torch.int32, device=dev)
    idx = torch.randint(0, S // bs, (B, Hq, 3), generator=g)
    idx[:, :, 2] = -1  # padding slot
    nb = S // bs
    mask = torch.zeros(B, Hq, 1, nb, dtype=torch.bool)
    for b in range(B):
        for h in range(Hq):
            for j in idx[b, h].tolist():
                if j >= 0:
                    mask[b, h, 0, j] = True
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    a = bsfa.forward_decode_paged(q, kp, vp, table, lens, block_indices=idx.to(dev))
    m = bsfa.forward_decode_paged(q, kp, vp, table, lens, mask.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(a, m)


@pytest.mark.parametrize("splits", (1, 4))
def test_decode_empty_sequences_and_heads_give_zero(splits):
    """Zero-length sequences and heads that select no block output exactly 0 (the closed
    form's empty case), with one split and with partials merged by the combine pass, for the
    contiguous and the paged cache; the other rows still match the oracle."""
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs, ps = 4, 8, 2, 300, 128, 64, 16
    print(f"decode empty rows splits={splits}", flush=True)
    g = torch.Generator().manual_seed(7700 + splits)
    per = (S + ps - 1) // ps
    cap = per * ps
    q = (torch.randn(B, Hq, 1, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    k = (torch.randn(B, Hkv, cap, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    v = (torch.randn(B, Hkv, cap, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    lens = torch.tensor([0, 300, 1, 0], dtype=torch.int32)
    nb = (cap + bs - 1) // bs
    mask = torch.rand((B, Hq, 1, nb), generator=g) < 0.5
    mask[:, :, :, 0] = True
    mask[1, 3] = False  # a head of a non-empty sequence with nothing selected
    mask[2, 5] = False
    table = torch.randperm(B * per, generator=g).view(B, per).to(torch.int32)
    kp = torch.zeros(B * per, ps, Hkv, D, dtype=torch.bfloat16)
    vp = torch.zeros(B * per, ps, Hkv, D, dtype=torch.bfloat16)
    for b in range(B):
        for j in range(per):
            kp[table[b, j]] = k[b, :, j * ps:(j + 1) * ps].transpose(0, 1)
            vp[table[b, j]] = v[b, :, j * ps:(j + 1) * ps].transpose(0, 1)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    contig = bsfa.forward_decode(q.to(dev), k.to(dev), v.to(dev), mask.to(dev),
                                 kv_lens=lens.to(dev), num_splits=splits)
    paged = bsfa.forward_decode_paged(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev),
                                      lens.to(dev), mask.to(dev), num_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(paged, contig)
    out = contig.cpu()
    assert (out[0] == 0).all() and (out[3] == 0).all()
    assert (out[1, 3] == 0).all() and (out[2, 5] == 0).all()
    assert torch.isfinite(out.float()).all()
    ref = orc.sparse_decode(to_np(q), to_np(k), to_np(v), mask.numpy(), bs, kv_lens=lens.numpy())
    assert_close_bf16(contig, ref, f"decode empty rows splits={splits}")
