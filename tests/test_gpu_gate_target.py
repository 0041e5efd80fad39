"""Gate-target kernel parity: block maxima and softmax targets vs the CPU oracle."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, require_gpu, to_np
from oracle import tasft_oracle as orc
from tasft_amd import workloads as wl
from tasft_amd.training import TASFTObjective, gate_target_from_qk

pytestmark = pytest.mark.gpu

RAW_RTOL = 1e-4
RAW_ATOL = 1e-6


def _gt(q, k, bs, **kw):
    out = gate_target_from_qk(q, k, bs, **kw)
    torch.cuda.synchronize()
    return out


CASES = [
    # B, Hq, Hkv, S, D, bs, causal
    (1, 4, 4, 512, 128, 64, True),
    (2, 8, 2, 1000, 128, 64, True),   # GQA, ragged
    (1, 4, 1, 300, 64, 32, False),    # non-causal, D=64
    (1, 2, 2, 384, 128, 128, True),   # bs=128 (block-64 maxima pooled 2x2)
    (2, 4, 2, 450, 64, 128, False),   # bs=128, non-causal, ragged, D=64
    (1, 4, 2, 300, 128, 128, True),   # bs=128 over an odd number of 64-token blocks
    (2, 4, 2, 1000, 128, 32, True),   # bs=32 as 32x32 tiles of the block-64 kernel, ragged
    (1, 3, 3, 333, 128, 32, True),    # bs=32, one head per workgroup, last 64-block half empty
    (2, 4, 2, 640, 64, 64, True),     # two query heads per KV head share the K tiles, D=64
    (1, 3, 3, 200, 128, 64, False),   # one head per workgroup, non-causal, ragged
    (1, 2, 1, 2000, 64, 32, True),    # flat groups of 63 x 63 > 1024: register-resident softmax
]


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs", "causal"), CASES)
def test_block_max_and_targets_match_oracle(B, Hq, Hkv, S, D, bs, causal):
    dev = require_gpu()
    q, k, _ = wl.qkv(wl.Shape(B, Hq, Hkv, S, D), 300 + S)
    qd, kd = q.to(dev), k.to(dev)
    raw_ref = orc.block_max(to_np(q), to_np(k), bs, causal, dtype=np.float64)
    raw = to_np(_gt(qd, kd, bs, causal=causal, normalize="none"))
    assert np.array_equal(np.isneginf(raw), np.isneginf(raw_ref))
    fin = np.isfinite(raw_ref)
    np.testing.assert_allclose(raw[fin], raw_ref[fin], rtol=RAW_RTOL, atol=RAW_ATOL)
    for norm in ("flat", "row"):
        got = _gt(qd, kd, bs, causal=causal, normalize=norm)
        ref = orc.normalize_block_max(raw_ref, norm)
        assert_close_bf16(got, ref, f"gate target {norm}")
        np.testing.assert_allclose(to_np(got), ref, rtol=1e-3, atol=1e-7)


@pytest.mark.parametrize(("bs", "S"), [(32, 256), (64, 256), (128, 256), (32, 2048)])
def test_clamp_temperature_variant(bs, S):
    dev = require_gpu()
    q, k, _ = wl.qkv(wl.Shape(1, 4, 4, S, 128), 77)
    # Scale the queries so some block maxima exceed the clamp.
    q = (q.float() * 2000).to(torch.bfloat16)
    got = _gt(q.to(dev), k.to(dev), bs, normalize="flat", temperature=2.0, clamp=50.0)
    raw_ref = orc.block_max(to_np(q), to_np(k), bs, True, dtype=np.float64)
    assert np.nanmax(raw_ref[np.isfinite(raw_ref)]) > 50.0
    ref = orc.normalize_block_max(raw_ref, "flat", temperature=2.0, clamp=50.0)
    np.testing.assert_allclose(to_np(got), ref, rtol=1e-3, atol=1e-7)


def test_matches_reference_dense_path_on_explicit_scores():
    """gate_target_from_qk == compute_gate_target(Q K^T * scale + triu(-inf))."""
    dev = require_gpu()
    q, k, _ = wl.qkv(wl.Shape(1, 4, 2, 256, 128), 88)
    got = _gt(q.to(dev), k.to(dev), 64)
    kk = k.float().repeat_interleave(2, 1)
    scores = (q.float() @ kk.transpose(-1, -2)) / math.sqrt(128)
    scores = scores + torch.full((256, 256), float("-inf")).triu(1)
    ref = TASFTObjective.compute_gate_target(scores, 64)
    torch.testing.assert_close(got.cpu(), ref, rtol=1e-3, atol=1e-7)


def test_config5_full_size_sampled_heads():
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[5]
    q, k, _ = wl.qkv(shape, 1005)
    got = to_np(_gt(q.to(dev), k.to(dev), 64))
    np.testing.assert_allclose(got.reshape(4, 32, -1).sum(-1), 1.0, rtol=1e-4)
    assert (got[..., np.triu(np.ones((64, 64), bool), 1)] == 0).all()
    for b, h in [(0, 0), (3, 31)]:
        ref = orc.gate_target_from_qk(to_np(q[b : b + 1, h : h + 1]), to_np(k[b : b + 1, h // 4 : h // 4 + 1]), 64)
        np.testing.assert_allclose(got[b, h], ref[0, 0], rtol=1e-3, atol=1e-7)


def test_config5_blocks_32_64_128_nest_by_2x2_max():
    """Block 128 merges each 64-block maximum into its 128-block by atomic max, and block 32
    writes the 32 x 32 tiles of the same block-64 kernel: at full size the block-64 raw
    maxima are exactly the 2x2 max of the block-32 ones, the block-128 maxima exactly the
    2x2 max of the block-64 ones (max is exact and order-free), and sampled heads match the
    oracle's block-32 and block-128 targets."""
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[5]
    q, k, _ = wl.qkv(shape, 1005)
    qd, kd = q.to(dev), k.to(dev)
    r64 = _gt(qd, kd, 64, normalize="none")
    r128 = _gt(qd, kd, 128, normalize="none")
    r32 = _gt(qd, kd, 32, normalize="none")
    B, H, nb, _ = r128.shape
    assert torch.equal(r128, r64.view(B, H, nb, 2, nb, 2).amax(dim=(3, 5)))
    assert torch.equal(r64, r32.view(B, H, 2 * nb, 2, 2 * nb, 2).amax(dim=(3, 5)))
    for bs, (b, h) in ((128, (2, 17)), (32, (1, 6))):
        got = to_np(_gt(qd, kd, bs))
        ref = orc.gate_target_from_qk(to_np(q[b : b + 1, h : h + 1]), to_np(k[b : b + 1, h // 4 : h // 4 + 1]), bs)
        np.testing.assert_allclose(got[b, h], ref[0, 0], rtol=1e-3, atol=1e-7)


MASK_CASES = [
    # B, Hq, Hkv, S, D, bs, form
    (2, 8, 2, 700, 128, 64, "padding_2d"),    # four heads per workgroup, ragged, key padding
    (2, 4, 2, 640, 64, 64, "binary_2d"),      # two heads per workgroup; the reference adds 1/0
    (2, 3, 3, 333, 128, 64, "hf_4d"),         # one head per workgroup, HF [B, 1, S, S] mask
    (1, 4, 2, 300, 128, 32, "per_head_4d"),   # block 32 (32 x 32 quarters), per-head mask
    (2, 8, 2, 700, 128, 32, "padding_2d"),    # block 32, key padding, 22 blocks (11 of 64)
    (1, 4, 2, 330, 64, 32, "hf_4d"),          # block 32, odd block count: mask read to 384
    (2, 2, 1, 400, 64, 128, "padding_2d"),    # block 128: block-64 maxima pooled 2x2
    (1, 4, 4, 333, 128, 128, "hf_4d"),        # block 128, odd block-64 count, HF mask
]


def _attention_mask(form, B, Hq, S, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.tensor([S] + [int(S * 0.6)] * (B - 1))
    keep = torch.arange(S)[None, :] < lens[:, None]
    if form == "padding_2d":
        return torch.zeros(B, S).masked_fill(~keep, float("-inf"))
    if form == "binary_2d":
        return keep.to(torch.int64)  # HF's 1 = attend / 0 = pad, added as-is by the reference
    if form == "hf_4d":
        causal = torch.ones(S, S, dtype=torch.bool).tril()
        allowed = causal[None] & keep[:, None, :]
        return torch.zeros(B, 1, S, S).masked_fill(~allowed[:, None], torch.finfo(torch.float32).min)
    return torch.randn(B, Hq, S, S, generator=g)


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs", "form"), MASK_CASES)
def test_attention_mask_matches_oracle(B, Hq, Hkv, S, D, bs, form):
    """Padded batches: the additive attention_mask of tasft_attention.py:445-449 is added to
    the scaled scores before the max-pool (raw maxima, flat and row targets)."""
    dev = require_gpu()
    print(f"gate target mask {form} B={B} Hq={Hq} S={S} D={D} bs={bs}", flush=True)
    q, k, _ = wl.qkv(wl.Shape(B, Hq, Hkv, S, D), 500 + S)
    q = (q.float() * math.sqrt(D)).to(torch.bfloat16)  # unit-scale scores
    mask = _attention_mask(form, B, Hq, S, 600 + S)
    qd, kd, md = q.to(dev), k.to(dev), mask.to(dev)
    m_np = mask.double().numpy()
    raw_ref = orc.block_max(to_np(q), to_np(k), bs, True, dtype=np.float64, attn_mask=m_np)
    raw = to_np(_gt(qd, kd, bs, normalize="none", attention_mask=md))
    assert np.array_equal(np.isneginf(raw), np.isneginf(raw_ref))
    fin = np.isfinite(raw_ref)
    np.testing.assert_allclose(raw[fin], raw_ref[fin], rtol=RAW_RTOL, atol=1e-5)
    for norm in ("flat", "row"):
        got = to_np(_gt(qd, kd, bs, normalize=norm, attention_mask=md))
        ref = orc.normalize_block_max(raw_ref, norm)
        np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-7)
    if form == "padding_2d":
        # The padded rows' targets differ from the unmasked ones (the mask matters).
        plain = to_np(_gt(qd, kd, bs))
        assert not np.allclose(plain[1], orc.normalize_block_max(raw_ref, "flat")[1], atol=1e-4)


def test_attention_mask_rejects_nan_and_bad_shapes():
    from tasft_amd.exceptions import KernelError, NaNDetectedError

    dev = require_gpu()
    q, k, _ = (t.to(dev) for t in wl.qkv(wl.Shape(1, 4, 2, 128, 128), 7))
    bad = torch.zeros(1, 128, device=dev)
    bad[0, 5] = float("nan")
    with pytest.raises(NaNDetectedError):
        gate_target_from_qk(q, k, 64, attention_mask=bad)
    with pytest.raises(KernelError, match="broadcast"):
        gate_target_from_qk(q, k, 64, attention_mask=torch.zeros(1, 1, 128, 100, device=dev))
