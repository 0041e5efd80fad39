"""Fused AttnGate parity: HIP logits vs the oracle, and bit-exact masks from identical logits.

Bar (north star): masks bit-exact when computed from identical fp32 logits, excluding
scores within 1e-6 of the threshold; logits compared separately with a tolerance.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import require_gpu, to_np
from oracle import tasft_oracle as orc
from tasft_amd import workloads as wl
from tasft_amd.modules import AttnGate

pytestmark = pytest.mark.gpu

LOGIT_ATOL = 1e-5
LOGIT_RTOL = 1e-4
TAU_BAND = 1e-6


def _gate(H, D, bs, hidden, causal=True, seed=0):
    torch.manual_seed(seed)
    return AttnGate(num_heads=H, head_dim=D, block_size=bs, gate_hidden_dim=hidden, is_causal=causal)


def _params(gate):
    return (gate.gate_proj_in.weight.detach().numpy(), gate.gate_proj_in.bias.detach().numpy(),
            gate.gate_proj_out.weight.detach().numpy())


def _check(gate, q, k, tau, causal, force_diagonal=False):
    dev = require_gpu()
    gd = gate.to(dev)
    with torch.no_grad():
        out = gd(q.to(dev), k.to(dev), threshold=tau, return_logits=True, force_diagonal=force_diagonal)
    torch.cuda.synchronize()
    gate.cpu()
    w_in, b_in, w_out = _params(gate)
    ref_logits = orc.gate_logits(to_np(q), to_np(k), w_in, b_in, w_out, gate.block_size, dtype=np.float64)
    logits = to_np(out.logits)
    np.testing.assert_allclose(logits, ref_logits, rtol=LOGIT_RTOL, atol=LOGIT_ATOL)
    taus = tau.cpu().numpy() if isinstance(tau, torch.Tensor) else tau
    soft_ref, hard_ref = orc.threshold_mask(logits, taus, causal)
    if force_diagonal:
        hard_ref = hard_ref | np.eye(hard_ref.shape[-1], dtype=bool)
    soft = to_np(out.soft_scores)
    np.testing.assert_allclose(soft, soft_ref, rtol=0, atol=2e-7)
    hard = out.hard_mask.cpu().numpy()
    t = np.asarray(taus, dtype=np.float32)
    t = t.reshape(1, -1, 1, 1) if t.ndim == 1 else t
    decisive = np.abs(soft_ref - t) > TAU_BAND
    if force_diagonal:
        decisive |= np.eye(hard.shape[-1], dtype=bool)
    assert np.array_equal(hard[decisive], hard_ref[decisive]), "hard mask differs from identical logits"
    if causal:
        up = np.triu(np.ones(soft.shape[-2:], bool), 1)
        assert (soft[..., up] == 0.0).all()
    assert out.sparsity_ratio == pytest.approx(1.0 - hard.mean(), abs=1e-9)
    return out


CASES = [
    # B, Hq, Hkv, S, D, bs, hidden, causal
    (2, 4, 4, 512, 128, 64, 32, True),
    (1, 8, 2, 1000, 128, 64, 128, True),   # GQA, ragged (padded last block)
    (2, 4, 4, 64, 32, 8, 32, True),        # reference test geometry (small_gate)
    (1, 4, 4, 30, 16, 8, 32, False),       # non-causal, ragged
    (1, 8, 8, 256, 64, 16, 48, True),      # odd hidden size
    (1, 2, 1, 777, 128, 48, 64, True),     # block size outside {32,64,128}
    (1, 4, 2, 700, 64, 64, 32, True),      # block 64, D=64, 11 blocks (partial pool chunk)
    (1, 4, 2, 1300, 128, 64, 200, False),  # block 64, 21 blocks, hidden > one staging tile
    (1, 4, 2, 1300, 128, 64, 64, False),   # block 64, non-causal, fused query-pool + pairwise
    (1, 2, 1, 9000, 128, 64, 32, True),    # 141 blocks: two 128-key groups per row
    (1, 4, 2, 1000, 128, 128, 64, True),   # block 128 streaming pool, ragged, one partial chunk
    (2, 4, 2, 2500, 64, 128, 48, False),   # block 128, D=64, non-causal, 20 blocks (two chunks)
    (1, 4, 2, 1000, 128, 32, 64, True),    # block 32 streaming pool, 32 blocks (two chunks)
    (2, 2, 2, 600, 64, 32, 32, False),     # block 32, D=64, non-causal, ragged partial chunk
]


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs", "hidden", "causal"), CASES)
def test_gate_matches_oracle(B, Hq, Hkv, S, D, bs, hidden, causal):
    gate = _gate(Hq, D, bs, hidden, causal, seed=S)
    q = wl.randn_bf16((B, Hq, S, D), S, scale=1.0)
    k = wl.randn_bf16((B, Hkv, S, D), S + 1, scale=1.0)
    _check(gate, q, k, 0.5, causal)


def test_threshold_edges_and_per_head_tau():
    gate = _gate(4, 32, 8, 32)
    q = wl.randn_bf16((2, 4, 32, 32), 1, scale=1.0)
    k = wl.randn_bf16((2, 4, 32, 32), 2, scale=1.0)
    out0 = _check(gate, q, k, 0.0, True)
    assert out0.hard_mask.all()  # 0 >= 0 holds in the zeroed upper triangle too
    out1 = _check(gate, q, k, 1.0 + 1e-7, True)
    assert not out1.hard_mask.any()
    assert out1.sparsity_ratio == pytest.approx(1.0)
    taus = torch.tensor([0.0, 0.49, 0.5, 0.51])
    _check(gate, q, k, taus, True)
    _check(gate, q, k, 0.6, True, force_diagonal=True)


def test_gqa_equals_expanded_k():
    dev = require_gpu()
    gate = _gate(8, 128, 64, 64).to(dev)
    q = wl.randn_bf16((1, 8, 512, 128), 3).to(dev)
    k = wl.randn_bf16((1, 2, 512, 128), 4).to(dev)
    with torch.no_grad():
        a = gate(q, k, return_logits=True)
        b = gate(q, k.repeat_interleave(4, dim=1), return_logits=True)
    torch.cuda.synchronize()
    assert torch.equal(a.logits, b.logits) and torch.equal(a.hard_mask, b.hard_mask)


def test_autograd_path_matches_kernel_and_has_gradients():
    dev = require_gpu()
    gate = _gate(4, 64, 16, 32).to(dev)
    q = wl.randn_bf16((1, 4, 128, 64), 5, scale=1.0).to(dev)
    k = wl.randn_bf16((1, 4, 128, 64), 6, scale=1.0).to(dev)
    with torch.no_grad():
        ref = gate(q, k, return_logits=True)
    out = gate(q, k, return_logits=True)  # parameters require grad -> differentiable path
    torch.testing.assert_close(out.logits.detach(), ref.logits, rtol=1e-4, atol=1e-5)
    out.soft_scores.sum().backward()
    for name, p in gate.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().sum() > 0, name


def test_config2_gate_full_size_sampled_heads():
    """Config 2 geometry: B=4, S=8192, 32/8 heads, hidden 128; heads sampled for the oracle."""
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[2]
    q, k, _ = wl.qkv(shape, 1002)
    gate = AttnGate(num_heads=32, head_dim=128, gate_hidden_dim=128)
    gate.load_state_dict(wl.gate_params(128, 128, 3002))
    gd = gate.to(dev)
    with torch.no_grad():
        out = gd(q.to(dev), k.to(dev), threshold=0.5, return_logits=True)
    torch.cuda.synchronize()
    gate.cpu()
    w_in, b_in, w_out = _params(gate)
    logits = to_np(out.logits)
    for b, h in [(0, 0), (2, 17), (3, 31)]:
        ref = orc.gate_logits(to_np(q[b : b + 1, h : h + 1]), to_np(k[b : b + 1, h // 4 : h // 4 + 1]),
                              w_in, b_in, w_out, 64, dtype=np.float64)[0, 0]
        np.testing.assert_allclose(logits[b, h], ref, rtol=LOGIT_RTOL, atol=LOGIT_ATOL)
    soft_ref, hard_ref = orc.threshold_mask(logits, 0.5, True)
    decisive = np.abs(soft_ref - 0.5) > TAU_BAND
    hard = out.hard_mask.cpu().numpy()
    assert np.array_equal(hard[decisive], hard_ref[decisive])


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "hidden"), [
    (4, 32, 8, 8192, 128, 128),  # config 2
    (1, 2, 1, 9000, 128, 32),    # two 128-key groups per row
    (2, 4, 2, 700, 64, 64),      # D = 64, partial last query chunk
])
def test_causal_rows_skip_matches_full_evaluation(B, Hq, Hkv, S, D, hidden):
    """Without logits, the causal gate evaluates only the key blocks a query chunk needs
    (the rest are exactly 0); with logits it evaluates every pair. Soft scores, the mask
    (per-head tau, forced diagonal) and the active count must agree bit for bit."""
    dev = require_gpu()
    gate = _gate(Hq, D, 64, hidden, True, seed=S + hidden).to(dev).requires_grad_(False)
    q = wl.randn_bf16((B, Hq, S, D), S + 7, scale=1.0).to(dev)
    k = wl.randn_bf16((B, Hkv, S, D), S + 8, scale=1.0).to(dev)
    taus = torch.linspace(0.3, 0.7, Hq, device=dev)
    with torch.no_grad():
        full = gate(q, k, threshold=taus, return_logits=True, force_diagonal=True)
        rows = gate(q, k, threshold=taus, force_diagonal=True)
    torch.cuda.synchronize()
    assert rows.logits is None
    assert torch.equal(rows.soft_scores, full.soft_scores)
    assert torch.equal(rows.hard_mask, full.hard_mask)
    assert rows.sparsity_ratio == full.sparsity_ratio
    assert rows.sparsity_ratio == pytest.approx(1.0 - full.hard_mask.double().mean().item(), abs=1e-12)


def test_fp32_inputs_run_the_reference_formula_and_fp16_the_kernel():
    """fp32 Q/K on the GPU evaluate the reference formula in fp32 and agree with the kernel on
    the same values; fp16 Q/K (the same values, exact in fp16 apart from a rare tiny one in
    fp16's subnormal range) run the kernel's fp16 instantiation and give the same logits."""
    dev = require_gpu()
    gate = _gate(8, 128, 64, 64).to(dev).requires_grad_(False)
    q = wl.randn_bf16((1, 8, 700, 128), 41, scale=1.0).to(dev)
    k = wl.randn_bf16((1, 2, 700, 128), 42, scale=1.0).to(dev)
    with torch.no_grad():
        hip = gate(q, k, return_logits=True)
        f32 = gate(q.float(), k.float(), return_logits=True)
        f16 = gate(q.half(), k.half(), return_logits=True)
    torch.cuda.synchronize()
    assert f32.soft_scores.dtype == torch.float32 and f16.soft_scores.dtype == torch.float32
    torch.testing.assert_close(f32.logits, hip.logits, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(f16.logits, hip.logits, rtol=1e-5, atol=1e-6)


def _gate_c_abi(gate, q, k, taus, workspace, flags=3):
    """tasft_gate_fwd through the C ABI on a caller-held workspace; returns (soft, mask, count)."""
    from tasft_amd import _native

    lib = _native.load_library()
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    nb = math.ceil(S / gate.block_size)
    dev = q.device
    w_in = gate.gate_proj_in.weight.detach().float().contiguous()
    b_in = gate.gate_proj_in.bias.detach().float().contiguous()
    w_out = gate.gate_proj_out.weight.detach().float().reshape(-1).contiguous()
    soft = torch.full((B, H, nb, nb), 7.0, dtype=torch.float32, device=dev)
    mask = torch.full((B, H, nb, nb), 9, dtype=torch.uint8, device=dev)
    count = torch.full((1,), -1, dtype=torch.int64, device=dev)
    rc = lib.tasft_gate_fwd(
        q.data_ptr(), k.data_ptr(), w_in.data_ptr(), b_in.data_ptr(), w_out.data_ptr(), taus.data_ptr(),
        soft.data_ptr(), None, mask.data_ptr(), count.data_ptr(), None, None, workspace.data_ptr(),
        workspace.numel(), B, H, Hkv, S, D, gate.block_size, gate.gate_hidden_dim,
        _native.strides(q), _native.strides(k), flags, _native.dtype_code(q.dtype, "gate"),
        _native.stream_handle(dev))
    assert rc == 0, lib.tasft_last_error()
    return soft, mask, count


def test_one_launch_gate_reuses_its_workspace():
    """The one-launch gate (block 64) on one workspace, first filled with 0xFF bytes (its
    completion counters included), twice in a row with different inputs: each call's outputs
    equal a fresh-workspace call's bit for bit, and the count (bit 63 clear) is the mask's sum."""
    from tasft_amd import _native

    dev = require_gpu()
    B, Hq, Hkv, S, D, hidden = 2, 8, 2, 2048, 128, 64
    gate = _gate(Hq, D, 64, hidden, True, seed=91).to(dev).requires_grad_(False)
    taus = torch.linspace(0.4, 0.6, Hq, device=dev)
    lib = _native.load_library()
    n = lib.tasft_gate_workspace_bytes(B, Hq, Hkv, S, D, 64, hidden)
    shared = torch.full((n,), 0xFF, dtype=torch.uint8, device=dev)
    for seed in (5, 6):
        q = wl.randn_bf16((B, Hq, S, D), seed, scale=1.0).to(dev)
        k = wl.randn_bf16((B, Hkv, S, D), seed + 50, scale=1.0).to(dev)
        soft, mask, count = _gate_c_abi(gate, q, k, taus, shared)
        fresh = _gate_c_abi(gate, q, k, taus, torch.zeros((n,), dtype=torch.uint8, device=dev))
        torch.cuda.synchronize()
        assert torch.equal(soft, fresh[0]) and torch.equal(mask, fresh[1])
        c = int(count.item())
        assert c >= 0 and c == int(mask.sum().item()) == int(fresh[2].item())
        with torch.no_grad():
            mod = gate(q, k, threshold=taus, force_diagonal=True)
        assert torch.equal(mod.hard_mask.to(torch.uint8), mask)


def test_one_launch_gate_wait_error_path():
    """With the diagnostic switch on, the key workgroups publish nothing: every query
    workgroup's bounded wait gives up (every workgroup still exits), its rows get NaN scores
    and no mask bit, bit 63 of the count is set and GateOutput.sparsity_ratio raises
    KernelError. Switched off again, the same call gives the normal result."""
    from tasft_amd import _native
    from tasft_amd.exceptions import KernelError

    dev = require_gpu()
    gate = _gate(4, 128, 64, 64, True, seed=17).to(dev).requires_grad_(False)
    q = wl.randn_bf16((1, 4, 1024, 128), 71, scale=1.0).to(dev)
    k = wl.randn_bf16((1, 2, 1024, 128), 72, scale=1.0).to(dev)
    with torch.no_grad():
        good = gate(q, k, threshold=0.5)
    good_sparsity = good.sparsity_ratio
    lib = _native.load_library()
    try:
        assert lib.tasft_gate_debug_wait_fault(1) == 0
        with torch.no_grad():
            bad = gate(q, k, threshold=0.5)
        torch.cuda.synchronize()
    finally:
        lib.tasft_gate_debug_wait_fault(0)
    assert torch.isnan(bad.soft_scores).all()
    assert not bad.hard_mask.any()
    with pytest.raises(KernelError, match="timed out"):
        _ = bad.sparsity_ratio
    with torch.no_grad():
        again = gate(q, k, threshold=0.5)
    assert torch.equal(again.soft_scores, good.soft_scores)
    assert torch.equal(again.hard_mask, good.hard_mask)
    assert again.sparsity_ratio == good_sparsity
