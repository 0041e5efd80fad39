"""fp16 inputs on the HIP kernels: the reference kernel and gate take fp16 as well as bf16
(``tasft/kernels/block_sparse_fa.py:228, 252`` are dtype-generic ``tl.dot``;
``tasft/modules/attn_gate.py:59`` accepts fp16).

Every kernel runs its fp16 instantiation (v_mfma_f32_32x32x16_f16, P and the output
rounded to fp16) on fp16-rounded inputs and is compared with the same CPU oracle as the
bf16 tests, under the fp16 bar (``helpers.bar``: max-abs 5e-3, mean-abs 5e-4, relative
5e-3, four times tighter than bf16's). ``tests/test_discriminating_inputs.py`` shows on
the CPU that this bar rejects uniform weights, a doubled scale and swapped query rows on
these cases while an fp16 emulation of the kernel arithmetic meets it.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import attn_inputs as ai
from helpers import assert_close_bf16, bar, require_gpu, to_np
from oracle import tasft_oracle as orc
from tasft_amd.kernels import BlockSparseFlashAttention
from tasft_amd.modules import AttnGate
from tasft_amd.training import gate_target_from_qk

pytestmark = pytest.mark.gpu

F16 = torch.float16
KINDS = ("unit", "peaky")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("case", ai.F16_PREFILL_CASES, ids=ai.case_id)
def test_f16_prefill_matches_oracle(case, kind):
    from test_gpu_prefill import _prefill_capi

    dev = require_gpu()
    B, Hq, Hkv, S, D, bs, causal, _dens, variant = case
    print(f"fp16 prefill {case} {kind}", flush=True)
    q, k, v, mask = ai.prefill_case_inputs(case, kind, F16)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    out = bsfa.forward(qd, kd, vd, md, causal=causal)
    torch.cuda.synchronize()
    assert out.dtype == F16
    ref = orc.attention_block_gather(to_np(q), to_np(k), to_np(v), mask.numpy(), bs, causal)
    assert_close_bf16(out, ref, f"fp16 prefill {case} {kind}", **bar(F16))
    if variant == "4w":
        # The same kernel without the persistent work queue gives the same bits.
        assert torch.equal(_prefill_capi(qd, kd, vd, md, bs, causal, workspace=None), out)


@pytest.mark.parametrize("case", ai.VARLEN_CASES[:2], ids=ai.case_id)
def test_f16_varlen_matches_oracle(case):
    dev = require_gpu()
    lens, _Hq, _Hkv, _D, bs, causal, _dens = case
    print(f"fp16 varlen {case}", flush=True)
    q, k, v, cu, mask = ai.varlen_case_inputs(case, "peaky", F16)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward_varlen(q.to(dev), k.to(dev), v.to(dev), mask.to(dev),
                              torch.tensor(cu, dtype=torch.int32), causal=causal)
    torch.cuda.synchronize()
    ref = orc.attention_varlen(to_np(q), to_np(k), to_np(v), cu, mask.numpy(), bs, causal)
    assert_close_bf16(out, ref, f"fp16 varlen {case}", **bar(F16))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("case", ai.F16_DECODE_CASES, ids=ai.case_id)
def test_f16_decode_matches_oracle(case, kind):
    dev = require_gpu()
    B, _Hq, _Hkv, S, _D, bs, _dens, splits = case
    print(f"fp16 decode {case} {kind}", flush=True)
    q, kc, vc, mask = ai.decode_case_inputs(case, kind, F16)
    lens = torch.randint(1, S + 1, (B,), generator=torch.Generator().manual_seed(S)).to(torch.int32)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward_decode(q.to(dev), kc.to(dev), vc.to(dev), mask.to(dev), kv_lens=lens,
                              num_splits=splits)
    torch.cuda.synchronize()
    assert out.dtype == F16
    ref = orc.sparse_decode(to_np(q), to_np(kc), to_np(vc), mask.numpy(), bs, kv_lens=lens.numpy())
    assert_close_bf16(out, ref, f"fp16 decode {case} {kind}", **bar(F16))
    assert (to_np(out)[0, 0] == 0).all()  # head (0, 0) selects nothing


@pytest.mark.parametrize("case", [ai.PAGED_CASES[0], ai.PAGED_CASES[2]], ids=ai.case_id)
def test_f16_paged_decode_matches_oracle(case):
    dev = require_gpu()
    bs, splits = case[5], case[7]
    print(f"fp16 paged decode {case}", flush=True)
    q, _k, _v, kp, vp, table, lens, mask = ai.paged_case_inputs(case, "peaky", F16)
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    out = bsfa.forward_decode_paged(q.to(dev), kp.to(dev), vp.to(dev), table.to(dev), lens.to(dev),
                                    mask.to(dev), num_splits=splits)
    torch.cuda.synchronize()
    ref = orc.sparse_decode_paged(to_np(q), to_np(kp), to_np(vp), table.numpy(), lens.numpy(),
                                  mask.numpy(), bs)
    assert_close_bf16(out, ref, f"fp16 paged decode {case}", **bar(F16))


def test_f16_dtype_mismatch_raises():
    from tasft_amd.exceptions import KernelError

    dev = require_gpu()
    q = torch.zeros(1, 2, 64, 64, dtype=F16, device=dev)
    k = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device=dev)
    bsfa = BlockSparseFlashAttention(block_size=64, min_sparsity_for_speedup=0.0)
    mask = torch.ones(1, 2, 1, 1, dtype=torch.bool, device=dev)
    with pytest.raises(KernelError, match="float16|bfloat16"):
        bsfa.forward(q, k, k, mask)
    with pytest.raises(KernelError, match="bf16 or fp16"):
        bsfa.forward(q.float(), k.float(), k.float(), mask)


GATE_CASES = [
    # B, Hq, Hkv, S, D, bs, hidden
    (2, 8, 2, 1000, 128, 64, 128),   # streaming pool kernel, GQA, ragged
    (1, 4, 4, 700, 64, 64, 48),      # streaming pool kernel, D=64
    (1, 4, 2, 300, 128, 32, 64),     # generic pool kernel
]


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs", "hidden"), GATE_CASES)
def test_f16_gate_matches_oracle(B, Hq, Hkv, S, D, bs, hidden):
    """fp16 Q/K run the HIP gate (fp32 arithmetic, fp32 scores) like bf16 ones."""
    dev = require_gpu()
    torch.manual_seed(S)
    gate = AttnGate(num_heads=Hq, head_dim=D, block_size=bs, gate_hidden_dim=hidden).to(dev)
    gate.requires_grad_(False)
    q, k, _ = ai.qkv("unit", (B, Hq, S, D), (B, Hkv, S, D), S, bs, dtype=F16)
    with torch.no_grad():
        out = gate(q.to(dev), k.to(dev), return_logits=True)
    torch.cuda.synchronize()
    assert out.soft_scores.dtype == torch.float32 and out.logits is not None
    gate.cpu()
    ref = orc.gate_logits(to_np(q), to_np(k), gate.gate_proj_in.weight.numpy(),
                          gate.gate_proj_in.bias.numpy(), gate.gate_proj_out.weight.numpy(), bs,
                          dtype=np.float64)
    np.testing.assert_allclose(to_np(out.logits), ref, rtol=1e-4, atol=1e-5)
    soft_ref, hard_ref = orc.threshold_mask(to_np(out.logits), 0.5, True)
    np.testing.assert_allclose(to_np(out.soft_scores), soft_ref, rtol=0, atol=2e-7)
    decisive = np.abs(soft_ref - 0.5) > 1e-6
    assert np.array_equal(out.hard_mask.cpu().numpy()[decisive], hard_ref[decisive])


def test_f16_gate_training_matches_torch_autograd():
    """fp16 Q/K through the HIP gate forward and backward against torch autograd of the
    reference formula (computed in fp32 from the same fp16 values)."""
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs, hidden = 2, 8, 2, 1000, 128, 64, 64
    torch.manual_seed(11)
    gate = AttnGate(num_heads=Hq, head_dim=D, block_size=bs, gate_hidden_dim=hidden).to(dev)
    q, k, _ = ai.qkv("unit", (B, Hq, S, D), (B, Hkv, S, D), 12, bs, dtype=F16)
    q, k = q.to(dev), k.to(dev)
    nb = math.ceil(S / bs)
    r = torch.randn(B, Hq, nb, nb, generator=torch.Generator().manual_seed(13)).to(dev)

    def run(path):
        gate.zero_grad(set_to_none=True)
        qq = q.clone().requires_grad_(True)
        kk = k.clone().requires_grad_(True)
        out = gate(qq, kk) if path == "hip" else gate._forward_torch(qq, kk, 0.5, False, False)
        (out.soft_scores.float() * r).sum().backward()
        grads = {n: p.grad.detach().clone() for n, p in gate.named_parameters()}
        grads["q"], grads["k"] = qq.grad.float(), kk.grad.float()
        return out, grads

    out_h, g_h = run("hip")
    out_t, g_t = run("torch")
    torch.cuda.synchronize()
    torch.testing.assert_close(out_h.soft_scores.detach(), out_t.soft_scores.detach().float(),
                               rtol=1e-5, atol=1e-6)
    for name, ref in g_t.items():
        err = float((g_h[name].float() - ref.float()).abs().max())
        scale = float(ref.abs().max())
        # Q/K gradients are stored in fp16 (one rounding, 2^-11 relative).
        assert err <= 2e-3 * scale + 1e-7, f"{name}: max err {err:.3e} vs max |grad| {scale:.3e}"


@pytest.mark.parametrize("masked", [False, True])
def test_f16_gate_target_matches_oracle(masked):
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs = 2, 8, 2, 1000, 128, 64
    q, k, _ = ai.qkv("unit", (B, Hq, S, D), (B, Hkv, S, D), 17, bs, dtype=F16)
    amask = None
    if masked:
        amask = torch.zeros(B, S)
        amask[1, 700:] = float("-inf")
        amask[0, :5] = -3.0
    raw = gate_target_from_qk(q.to(dev), k.to(dev), bs, normalize="none",
                              attention_mask=None if amask is None else amask.to(dev))
    torch.cuda.synchronize()
    raw_ref = orc.block_max(to_np(q), to_np(k), bs, True, dtype=np.float64,
                            attn_mask=None if amask is None else amask.numpy())
    raw = to_np(raw)
    assert np.array_equal(np.isneginf(raw), np.isneginf(raw_ref))
    fin = np.isfinite(raw_ref)
    np.testing.assert_allclose(raw[fin], raw_ref[fin], rtol=1e-4, atol=1e-5)
