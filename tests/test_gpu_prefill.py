"""Prefill kernel parity: HIP (through the C ABI) vs the CPU oracle on identical inputs.

Bar: max-abs <= 2e-2 and mean-abs <= 2e-3 against the fp32 oracle on the same bf16
inputs (tests/helpers.py). Rows with no active key must be exactly 0.
"""
from __future__ import annotations

import math
import warnings

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import attn_inputs as ai
from helpers import assert_close_bf16, require_gpu, to_np
from oracle import tasft_oracle as orc
from tasft_amd import workloads as wl
from tasft_amd.kernels import BlockSparseFlashAttention

pytestmark = pytest.mark.gpu


def _run(q, k, v, mask, bs, causal):
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward(q, k, v, mask, causal=causal)
    torch.cuda.synchronize()
    return out


def _inputs(B, Hq, Hkv, S, D, seed):
    shape = wl.Shape(B, Hq, Hkv, S, D)
    return wl.qkv(shape, seed)


def test_config1_matches_oracle():
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[1]
    q, k, v = wl.qkv(shape, 1001)
    mask = wl.bernoulli_causal_mask(shape, 0.2, 2001)
    out = _run(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), shape.block, True)
    ref = orc.attention_block_gather(to_np(q), to_np(k), to_np(v), mask.numpy(), shape.block, True)
    assert_close_bf16(out, ref, "config 1 prefill")


CASES = [
    # B, Hq, Hkv, S, D, bs, causal, density
    (2, 4, 4, 256, 128, 64, True, 0.5),     # MHA (reference layout)
    (1, 8, 2, 1000, 128, 64, True, 0.4),    # GQA, ragged S
    (1, 4, 1, 300, 64, 32, False, 0.5),     # non-causal, D=64, bs=32
    (1, 2, 2, 384, 128, 128, True, 0.6),    # bs=128
    (1, 7, 1, 520, 128, 64, True, 0.3),     # G=7 (Qwen grouping), ragged
    (2, 4, 2, 192, 64, 128, False, 0.5),    # non-causal, bs=128, D=64, partial last block
    (1, 4, 2, 100, 128, 32, True, 1.0),     # all-true causal
]


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs", "causal", "density"), CASES)
def test_prefill_shapes_match_oracle(B, Hq, Hkv, S, D, bs, causal, density):
    dev = require_gpu()
    seed = 17 + S + Hq
    q, k, v = _inputs(B, Hq, Hkv, S, D, seed)
    nb = math.ceil(S / bs)
    g = torch.Generator().manual_seed(seed)
    mask = torch.rand((B, Hq, nb, nb), generator=g) < density
    out = _run(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), bs, causal)
    ref = orc.attention_dense_masked(to_np(q), to_np(k), to_np(v), mask.numpy(), bs, causal)
    assert_close_bf16(out, ref, f"prefill {B}x{Hq}/{Hkv}x{S}x{D} bs={bs} causal={causal}")


def test_empty_rows_are_exact_zero():
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs = 1, 4, 2, 512, 128, 64
    q, k, v = _inputs(B, Hq, Hkv, S, D, 5)
    nb = S // bs
    mask = torch.ones((B, Hq, nb, nb), dtype=torch.bool)
    mask[0, 1, 3, :] = False          # fully empty row
    mask[0, 2, 5, :6] = False         # only blocks above the diagonal remain -> empty under causal
    out = _run(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), bs, True)
    o = out.cpu()
    assert (o[0, 1, 3 * bs : 4 * bs] == 0).all()
    assert (o[0, 2, 5 * bs : 6 * bs] == 0).all()
    ref = orc.attention_dense_masked(to_np(q), to_np(k), to_np(v), mask.numpy(), bs, True)
    assert_close_bf16(out, ref, "empty rows")


def test_all_true_mask_equals_sdpa_fp32():
    dev = require_gpu()
    q, k, v = _inputs(2, 8, 2, 320, 128, 9)
    mask = torch.ones((2, 8, 5, 5), dtype=torch.bool)
    out = _run(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 64, True)
    kk, vv = k.float().repeat_interleave(4, 1), v.float().repeat_interleave(4, 1)
    ref = F.scaled_dot_product_attention(q.float(), kk, vv, is_causal=True).numpy()
    assert_close_bf16(out, ref, "all-true mask vs SDPA")


def test_strided_hf_layout_inputs():
    """Q/K/V as transposed views of [B, S, H, D] (the HF projection layout), no copies."""
    dev = require_gpu()
    B, S, Hq, Hkv, D = 2, 256, 8, 2, 128
    g = torch.Generator().manual_seed(21)
    base_q = (torch.randn((B, S, Hq, D), generator=g) / math.sqrt(D)).to(torch.bfloat16)
    base_k = (torch.randn((B, S, Hkv, D), generator=g) / math.sqrt(D)).to(torch.bfloat16)
    base_v = (torch.randn((B, S, Hkv, D), generator=g) / math.sqrt(D)).to(torch.bfloat16)
    q, k, v = (t.to(dev).transpose(1, 2) for t in (base_q, base_k, base_v))
    assert not q.is_contiguous()
    mask = torch.rand((B, Hq, 4, 4), generator=g) < 0.5
    out = _run(q, k, v, mask.to(dev), 64, True)
    ref = orc.attention_dense_masked(to_np(q), to_np(k), to_np(v), mask.numpy(), 64, True)
    assert_close_bf16(out, ref, "strided inputs")


@pytest.mark.parametrize("dtype", [torch.bool, torch.uint8, torch.int32])
def test_mask_dtypes(dtype):
    dev = require_gpu()
    q, k, v = _inputs(1, 4, 4, 192, 128, 31)
    g = torch.Generator().manual_seed(31)
    mask = torch.rand((1, 4, 3, 3), generator=g) < 0.6
    out = _run(q.to(dev), k.to(dev), v.to(dev), mask.to(dtype).to(dev), 64, True)
    ref = orc.attention_dense_masked(to_np(q), to_np(k), to_np(v), mask.numpy(), 64, True)
    assert_close_bf16(out, ref, f"mask dtype {dtype}")


def test_low_sparsity_policy_falls_back_to_dense_with_warning():
    dev = require_gpu()
    q, k, v = (t.to(dev) for t in _inputs(1, 4, 4, 128, 128, 3))
    mask = torch.ones((1, 4, 2, 2), dtype=torch.bool, device=dev)
    bsfa = BlockSparseFlashAttention(block_size=64, min_sparsity_for_speedup=0.5)
    with pytest.warns(UserWarning, match="dense fallback"):
        out = bsfa.forward(q, k, v, mask, causal=True)
    ref = F.scaled_dot_product_attention(q.float().cpu(), k.float().cpu(), v.float().cpu(), is_causal=True)
    assert_close_bf16(out, ref.numpy(), "dense fallback")


def _sampled_parity(cfg, mask, seed, heads, rows=None):
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[cfg]
    q, k, v = wl.qkv(shape, seed)
    out = _run(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), shape.block, True).cpu()
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    ref = orc.attention_block_gather(qn, kn, vn, mask.numpy(), shape.block, True, heads=heads)
    for b, h in heads:
        assert_close_bf16(out[b, h], ref[b, h], f"config {cfg} head ({b},{h})")
    assert torch.isfinite(out.float()).all()


def test_config2_gate_chain_full_size_sampled_heads():
    """The launch the bench times: the config-2 gate with per-head tau (80% causal
    sparsity) and the diagonal forced on, then the prefill under its mask. The mask is
    checked against the oracle's threshold of the kernel's own logits (every head), the
    prefill against the oracle on sampled heads, on the benchmark inputs and again on
    unit-scale inputs under the same mask."""
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[2]
    nb = shape.nb
    q, k, v = wl.qkv(shape, 1002)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    gate, taus = wl.config2_gate(dev, qd, kd)
    with torch.no_grad():
        g = gate(qd, kd, threshold=taus, force_diagonal=True, return_logits=True)
    torch.cuda.synchronize()
    logits = to_np(g.logits)
    t = taus.cpu().numpy()
    soft_ref, hard_ref = orc.threshold_mask(logits, t, True)
    hard_ref = hard_ref | np.eye(nb, dtype=bool)
    decisive = (np.abs(soft_ref - t.reshape(1, -1, 1, 1)) > 1e-6) | np.eye(nb, dtype=bool)
    hard = g.hard_mask.cpu().numpy()
    assert np.array_equal(hard[decisive], hard_ref[decisive])
    n_exec = int(np.count_nonzero(hard & np.tril(np.ones((nb, nb), dtype=bool))))
    n_causal = shape.batch * shape.q_heads * nb * (nb + 1) // 2
    assert abs((1.0 - n_exec / n_causal) - 0.8) < 0.005
    mask = g.hard_mask
    heads = [(0, 0), (1, 13), (3, 31)]
    out = _run(qd, kd, vd, mask, shape.block, True).cpu()
    ref = orc.attention_block_gather(to_np(q), to_np(k), to_np(v), hard, shape.block, True, heads=heads)
    for b, h in heads:
        assert_close_bf16(out[b, h], ref[b, h], f"config 2 head ({b},{h})")
    assert torch.isfinite(out.float()).all()
    del out
    qu, ku, vu = ai.qkv("unit", tuple(q.shape), tuple(k.shape), 4002, shape.block)
    out = _run(qu.to(dev), ku.to(dev), vu.to(dev), mask, shape.block, True).cpu()
    ref = orc.attention_block_gather(to_np(qu), to_np(ku), to_np(vu), hard, shape.block, True,
                                     heads=heads)
    for b, h in heads:
        assert_close_bf16(out[b, h], ref[b, h], f"config 2 unit-scale head ({b},{h})")


def test_config4_full_size_sampled_heads():
    """Config 4 (Qwen-2.5-7B: 28/4 heads, G=7, rows of up to 256 key blocks, i.e. four
    64-byte mask chunks per row) at full size, on the benchmark inputs and again on
    unit-scale inputs under the same mask, where the softmax is far from uniform. The
    sampled heads include the first and last query head of a KV group."""
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[4]
    mask, _ = wl.qwen_mask(shape, 2004)
    heads = [(0, 0), (0, 6), (1, 13), (1, 27)]
    _sampled_parity(4, mask, 1004, heads=heads)
    q, k, v = wl.qkv(shape, 1004)
    qu, ku, vu = ai.qkv("unit", tuple(q.shape), tuple(k.shape), 4004, shape.block)
    del q, k, v
    out = _run(qu.to(dev), ku.to(dev), vu.to(dev), mask.to(dev), shape.block, True).cpu()
    ref = orc.attention_block_gather(to_np(qu), to_np(ku), to_np(vu), mask.numpy(), shape.block,
                                     True, heads=heads)
    for b, h in heads:
        assert_close_bf16(out[b, h], ref[b, h], f"config 4 unit-scale head ({b},{h})")


def _prefill_capi(q, k, v, mask, bs, causal, workspace=None):
    """tasft_bsfa_prefill_fwd called directly (``workspace`` None: one workgroup per row)."""
    import ctypes

    from tasft_amd import _native

    B, Hq, S, D = q.shape
    lib = _native.load_library()
    out = torch.empty_like(q)
    m8 = mask.view(torch.uint8)
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel())
    rc = lib.tasft_bsfa_prefill_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), m8.data_ptr(), ws_ptr, ws_bytes,
        B, Hq, k.shape[1], S, D, bs, _native.strides(q), _native.strides(k), _native.strides(v),
        _native.strides(out), _native.strides(m8), ctypes.c_float(1.0 / math.sqrt(D)),
        1 if causal else 0, _native.dtype_code(q.dtype, "prefill"), _native.stream_handle(q.device))
    _native.check(rc, "tasft_bsfa_prefill_fwd")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kind", ("unit", "peaky"))
@pytest.mark.parametrize("case", ai.PREFILL_CASES, ids=ai.case_id)
def test_prefill_discriminating_inputs(case, kind):
    """Scores far from uniform (unit scale; peaky keys that move the running maximum):
    pins QK^T, the exp2 scale, max tracking and the lazy rescale of every prefill kernel.
    The four-wave kernel runs with its persistent queue (the Python path) and without."""
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs, causal, _dens, variant = case
    print(f"prefill discriminating {case} {kind}", flush=True)
    q, k, v, mask = ai.prefill_case_inputs(case, kind)
    ref = orc.attention_block_gather(to_np(q), to_np(k), to_np(v), mask.numpy(), bs, causal)
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    out = _run(qd, kd, vd, md, bs, causal)
    assert_close_bf16(out, ref, f"prefill {variant} {kind}")
    if variant == "4w":
        direct = _prefill_capi(qd, kd, vd, md, bs, causal)
        assert_close_bf16(direct, ref, f"prefill {variant} {kind} (no work queue)")
        assert torch.equal(direct, out)


@pytest.mark.parametrize("kind", ("unit", "peaky"))
@pytest.mark.parametrize("case", ai.VARLEN_CASES, ids=ai.case_id)
def test_prefill_varlen_discriminating_inputs(case, kind):
    dev = require_gpu()
    lens, Hq, Hkv, D, bs, causal, _dens = case
    print(f"varlen discriminating {case} {kind}", flush=True)
    q, k, v, cu, mask = ai.varlen_case_inputs(case, kind)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward_varlen(q.to(dev), k.to(dev), v.to(dev), mask.to(dev),
                              torch.tensor(cu, dtype=torch.int32), causal=causal)
    torch.cuda.synchronize()
    ref = orc.attention_varlen(to_np(q), to_np(k), to_np(v), cu, mask.numpy(), bs, causal)
    assert_close_bf16(out, ref, f"varlen {lens} {kind}")


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs"), [
    (2, 16, 4, 2048, 64, 64),    # 8 KV groups: per-XCD partitions of the work queue
    (2, 6, 3, 1500, 64, 64),     # 6 KV groups: one partition, ragged
    (2, 16, 4, 2048, 128, 64),   # two-wave kernel: the workspace is left unused
    (1, 8, 2, 1024, 128, 128),   # block 128 on the two-wave kernel
    (2, 16, 4, 1500, 64, 128),   # block 128 on the four-wave kernel's work queue, ragged
])
def test_persistent_queue_is_bit_identical(B, Hq, Hkv, S, D, bs):
    """The persistent work queue (workspace given; head dim 64 at block 64 or 128) must not
    change any output bit against one workgroup per row."""
    dev = require_gpu()
    q, k, v = ai.qkv("unit", (B, Hq, S, D), (B, Hkv, S, D), 4242 + S + D, bs)
    shape = wl.Shape(B, Hq, Hkv, S, D, bs)
    mask = wl.bernoulli_causal_mask(shape, 0.15, 5151 + S)
    mask[0, 1, -3:, :] = True   # whole rows lit, as a gate can produce
    mask[B - 1, Hq - 1, 5, :] = True
    q, k, v, mask = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    out_ws = _run(q, k, v, mask, bs, True)  # the Python path passes a workspace
    out = _prefill_capi(q, k, v, mask, bs, True)
    assert torch.equal(out, out_ws)
    ref = orc.attention_block_gather(to_np(q.cpu()), to_np(k.cpu()), to_np(v.cpu()),
                                     mask.cpu().numpy(), bs, True)
    assert_close_bf16(out_ws, ref, "persistent prefill")


# ----------------------------------------------------------------------------- varlen
def _packed(lens, Hq, Hkv, D, seed, pad=5):
    """Packed bf16 q [T, Hq, D], k/v [T, Hkv, D] (T = sum(lens) + pad) and cu_seqlens."""
    g = torch.Generator().manual_seed(seed)
    T = sum(lens) + pad
    q = (torch.randn(T, Hq, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    k = (torch.randn(T, Hkv, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    v = (torch.randn(T, Hkv, D, generator=g) / math.sqrt(D)).to(torch.bfloat16)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return q, k, v, cu


VARLEN_CASES = [
    # lengths, Hq, Hkv, D, bs, causal, density
    ([100, 0, 257, 64, 1], 8, 2, 128, 64, True, 0.5),   # two-wave kernel; empty and 1-token
    ([300, 45, 128], 4, 4, 64, 64, True, 0.5),          # four-wave kernel (D=64)
    ([130, 77], 4, 2, 64, 32, False, 0.6),              # generic kernel, non-causal
    ([513, 200], 7, 1, 128, 128, True, 0.4),            # bs=128, G=7
    ([64, 1, 95, 700], 16, 2, 128, 32, True, 0.3),      # G=8, bs=32, block-aligned and 1-token
    ([333, 334], 8, 1, 64, 64, False, 0.7),             # non-causal four-wave kernel
]


@pytest.mark.parametrize(("lens", "Hq", "Hkv", "D", "bs", "causal", "density"), VARLEN_CASES)
def test_prefill_varlen_matches_oracle(lens, Hq, Hkv, D, bs, causal, density):
    dev = require_gpu()
    print(f"varlen lens={lens} Hq={Hq} Hkv={Hkv} D={D} bs={bs} causal={causal}", flush=True)
    q, k, v, cu = _packed(lens, Hq, Hkv, D, 6100 + sum(lens))
    nb = math.ceil(max(lens) / bs)
    g = torch.Generator().manual_seed(6200 + sum(lens))
    mask = torch.rand((len(lens), Hq, nb, nb), generator=g) < density
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward_varlen(q.to(dev), k.to(dev), v.to(dev), mask.to(dev),
                              torch.tensor(cu, dtype=torch.int32), causal=causal)
    torch.cuda.synchronize()
    ref = orc.attention_varlen(to_np(q), to_np(k), to_np(v), cu, mask.numpy(), bs, causal)
    assert_close_bf16(out, ref, f"varlen prefill {lens}")
    assert (out[cu[-1]:] == 0).all()
    # cu_seqlens on the device (no host round trip): the same rows, and the uncovered ones
    # zeroed on the device. The freed NaN block makes a stale output visible.
    poison = torch.full_like(out, float("nan"))
    del poison
    out_d = bsfa.forward_varlen(q.to(dev), k.to(dev), v.to(dev), mask.to(dev),
                                torch.tensor(cu, dtype=torch.int32, device=dev),
                                max_seqlen=max(max(lens), 1), causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(out_d[:cu[-1]], out[:cu[-1]])
    assert (out_d[cu[-1]:] == 0).all()


def test_prefill_varlen_one_sequence_is_bit_identical_to_forward():
    """One packed sequence runs the same kernel arithmetic as the dense call on the
    [1, H, T, D] view of the same memory (the reference's flat-token layout)."""
    dev = require_gpu()
    T, Hq, Hkv, D, bs = 1000, 8, 2, 128, 64
    q, k, v, cu = _packed([T], Hq, Hkv, D, 6300, pad=0)
    mask = wl.bernoulli_causal_mask(wl.Shape(1, Hq, Hkv, T, D, bs), 0.3, 6301)
    q, k, v, mask = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    dense = bsfa.forward(q.transpose(0, 1)[None], k.transpose(0, 1)[None],
                         v.transpose(0, 1)[None], mask, causal=True)
    # cu_seqlens on the device: no host check, max_seqlen given.
    packed = bsfa.forward_varlen(q, k, v, mask, torch.tensor(cu, dtype=torch.int32, device=dev),
                                 max_seqlen=T, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(packed, dense[0].transpose(0, 1))


def _expand128(mask128: torch.Tensor, nb64: int) -> torch.Tensor:
    """A block-128 mask as the equivalent block-64 mask: every 128-token block is its four
    64-token quarters."""
    return mask128.repeat_interleave(2, -1).repeat_interleave(2, -2)[..., :nb64, :nb64].contiguous()


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "causal"), [
    (1, 8, 2, 1000, 128, True),    # two-wave kernel, ragged: the last 128-block is partial
    (2, 4, 2, 1500, 64, True),     # four-wave kernel through its persistent work queue
    (1, 4, 4, 777, 128, False),    # non-causal, ragged
])
def test_block128_is_bit_identical_to_expanded_block64(B, Hq, Hkv, S, D, causal):
    """A block-128 mask runs on the block-64 kernels through the mask index shift; the
    output must equal, bit for bit, the block-64 launch on the 2x2-expanded mask."""
    dev = require_gpu()
    print(f"block128 bit identity B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal}", flush=True)
    q, k, v = ai.qkv("unit", (B, Hq, S, D), (B, Hkv, S, D), 8800 + S + D, 128)
    nb128, nb64 = math.ceil(S / 128), math.ceil(S / 64)
    mask = ai.random_mask((B, Hq, nb128, nb128), 0.4, 8900 + S)
    mask[0, 0, -1, :] = True
    q, k, v, mask = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    a = _run(q, k, v, mask, 128, causal)
    b = _run(q, k, v, _expand128(mask, nb64), 64, causal)
    assert torch.equal(a, b)


def test_block128_varlen_is_bit_identical_to_expanded_block64():
    dev = require_gpu()
    lens, Hq, Hkv, D = [513, 200, 64, 1], 7, 1, 128
    q, k, v, cu = ai.packed_qkv("unit", lens, Hq, Hkv, D, 9010, 128)
    nb128, nb64 = math.ceil(max(lens) / 128), math.ceil(max(lens) / 64)
    mask = ai.random_mask((len(lens), Hq, nb128, nb128), 0.5, 9011)
    bsfa128 = BlockSparseFlashAttention(block_size=128, min_sparsity_for_speedup=0.0)
    bsfa64 = BlockSparseFlashAttention(block_size=64, min_sparsity_for_speedup=0.0)
    cu_t = torch.tensor(cu, dtype=torch.int32)
    q, k, v, mask = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    a = bsfa128.forward_varlen(q, k, v, mask, cu_t, causal=True)
    b = bsfa64.forward_varlen(q, k, v, _expand128(mask, nb64), cu_t, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
