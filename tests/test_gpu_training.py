"""Gate training on the HIP kernels: the fused KL gate loss and the AttnGate backward.

* ``tasft_gate_kl_fwd`` against the oracle's KL loss and gradient (pinned to F.kl_div with
  "batchmean" and to torch autograd).
* ``gate_loss_from_qk`` against the reference composition
  ``compute_gate_loss(gate, compute_gate_target(scores))`` on explicitly built fp32 scores
  (with and without an attention mask), value and gradient.
* ``AttnGate`` training through ``tasft_gate_bwd`` against torch autograd of the reference
  formula (the torch path of the same module) for every parameter and for Q and K.
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
from tasft_amd.training import TASFTObjective, gate_loss_from_qk, gate_target_from_qk

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("NB", [20, 37, 128, 160])
def test_gate_kl_kernel_matches_oracle(NB):
    """NB 37 and 128 (16384 entries per (b, head), the largest) run the register-resident
    kernel; NB 160 runs the streaming one."""
    from tasft_amd.training.objectives import _GateKL

    dev = require_gpu()
    g = torch.Generator().manual_seed(31 + NB)
    B, H = 3, 5
    soft = torch.sigmoid(torch.randn(B, H, NB, NB, generator=g)) * torch.ones(NB, NB).tril()
    raw = torch.randn(B, H, NB, NB, generator=g) * 4
    target = torch.softmax(raw.view(B, H, -1), -1).view(B, H, NB, NB)
    target[0, 1, :3] = 0.0
    sd = soft.to(dev).requires_grad_(True)
    loss = _GateKL.apply(sd, target.to(dev))
    loss.backward()
    torch.cuda.synchronize()
    ref = orc.gate_kl_loss(soft.double().numpy(), target.double().numpy())
    assert float(loss.detach()) == pytest.approx(ref, rel=1e-5)
    np.testing.assert_allclose(to_np(sd.grad), orc.gate_kl_grad(soft.double().numpy(), target.double().numpy()),
                               rtol=1e-4, atol=1e-10)


def _explicit_scores(q, k, scale, mask=None):
    g = q.shape[1] // k.shape[1]
    kk = k.float().repeat_interleave(g, 1)
    s = (q.float() @ kk.transpose(-1, -2)) * scale
    n = q.shape[2]
    s = s + torch.full((n, n), float("-inf"), device=q.device).triu(1)
    if mask is not None:
        s = s + (mask[:, None, None, :] if mask.ndim == 2 else mask)
    return s


@pytest.mark.parametrize("masked", [False, True])
def test_gate_loss_from_qk_matches_reference_composition(masked):
    dev = require_gpu()
    B, Hq, Hkv, S, D, bs = 2, 8, 2, 700, 128, 64
    q = wl.randn_bf16((B, Hq, S, D), 61, scale=1.0).to(dev)
    k = wl.randn_bf16((B, Hkv, S, D), 62, scale=1.0).to(dev)
    mask = None
    if masked:
        mask = torch.zeros(B, S, device=dev)
        mask[1, 500:] = float("-inf")
    torch.manual_seed(5)
    gate = AttnGate(num_heads=Hq, head_dim=D, block_size=bs, gate_hidden_dim=64).to(dev)
    with torch.no_grad():
        soft = gate(q, k).soft_scores
    s1 = soft.clone().requires_grad_(True)
    fused = gate_loss_from_qk(s1, q, k, bs, attention_mask=mask)
    fused.backward()
    s2 = soft.clone().requires_grad_(True)
    scores = _explicit_scores(q, k, 1.0 / math.sqrt(D), mask)
    ref = TASFTObjective.compute_gate_loss(s2, TASFTObjective.compute_gate_target(scores, bs))
    ref.backward()
    torch.cuda.synchronize()
    assert float(fused.detach()) == pytest.approx(float(ref.detach()), rel=1e-4)
    # The target differs from the explicit fp32 one by the bf16-MFMA score rounding.
    torch.testing.assert_close(s1.grad, s2.grad, rtol=5e-3, atol=1e-4 * float(s2.grad.abs().max()))


GATE_CASES = [
    # B, Hq, Hkv, S, D, bs, hidden, causal, q_grad
    (2, 8, 2, 1000, 128, 64, 128, True, False),   # GQA, ragged, fast pool kernel
    (1, 4, 4, 700, 64, 64, 48, True, True),       # D=64, hidden not a multiple of 64, Q/K grads
    (2, 4, 2, 300, 128, 32, 200, False, True),    # generic pool kernel, non-causal, two unit rounds
    (1, 2, 1, 2100, 128, 64, 32, True, False),    # 33 blocks: partial last tile
    (4, 8, 4, 4096, 64, 64, 64, True, False),     # weight gradients split over K (8 and 4 chunks)
]


@pytest.mark.parametrize(("B", "Hq", "Hkv", "S", "D", "bs", "hidden", "causal", "qk_grad"), GATE_CASES)
def test_attn_gate_hip_backward_matches_torch_autograd(B, Hq, Hkv, S, D, bs, hidden, causal, qk_grad):
    dev = require_gpu()
    print(f"gate backward B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} bs={bs} hid={hidden}", flush=True)
    torch.manual_seed(S + hidden)
    gate = AttnGate(num_heads=Hq, head_dim=D, block_size=bs, gate_hidden_dim=hidden,
                    is_causal=causal).to(dev)
    q = wl.randn_bf16((B, Hq, S, D), S, scale=1.0).to(dev)
    k = wl.randn_bf16((B, Hkv, S, D), S + 1, scale=1.0).to(dev)
    nb = math.ceil(S / bs)
    r = torch.randn(B, Hq, nb, nb, generator=torch.Generator().manual_seed(S)).to(dev)

    def run(path):
        gate.zero_grad(set_to_none=True)
        qq = q.clone().requires_grad_(qk_grad)
        kk = k.clone().requires_grad_(qk_grad)
        if path == "hip":
            out = gate(qq, kk)
        else:
            out = gate._forward_torch(qq, kk, 0.5, False, False)
        (out.soft_scores * r).sum().backward()
        grads = {n: p.grad.detach().clone() for n, p in gate.named_parameters()}
        if qk_grad:
            grads["q"], grads["k"] = qq.grad.float(), kk.grad.float()
        return out, grads

    out_h, g_h = run("hip")
    out_t, g_t = run("torch")
    torch.cuda.synchronize()
    assert out_h.soft_scores.requires_grad
    torch.testing.assert_close(out_h.soft_scores.detach(), out_t.soft_scores.detach(), rtol=1e-5, atol=1e-6)
    for name, ref in g_t.items():
        got = g_h[name]
        scale = float(ref.abs().max())
        err = float((got.float() - ref.float()).abs().max())
        assert err <= 2e-3 * scale + 1e-7, f"{name}: max err {err:.3e} vs max |grad| {scale:.3e}"


def test_gate_training_step_config2_scale():
    """One gate training step at config-2 scale (B=4, S=8192, 32/8 heads, hidden 128):
    HIP gate forward + fused KL loss + HIP backward against the torch formula's autograd
    gradients of the same loss."""
    dev = require_gpu()
    shape = wl.CONFIG_SHAPES[2]
    q, k, _ = wl.qkv(shape, 1002)
    q = (q.float() * math.sqrt(128)).to(torch.bfloat16).to(dev)  # unit-scale scores
    k = (k.float() * math.sqrt(128)).to(torch.bfloat16).to(dev)
    gate = AttnGate(num_heads=32, head_dim=128, gate_hidden_dim=128)
    gate.load_state_dict(wl.gate_params(128, 128, 3002))
    gate = gate.to(dev)
    target = gate_target_from_qk(q, k, 64)

    gate.zero_grad(set_to_none=True)
    out = gate(q, k)
    loss = gate_loss_from_qk(out.soft_scores, q, k, 64)
    loss.backward()
    g_hip = {n: p.grad.detach().clone() for n, p in gate.named_parameters()}
    gate.zero_grad(set_to_none=True)
    out_t = gate._forward_torch(q, k, 0.5, False, False)
    loss_t = TASFTObjective.compute_gate_loss(out_t.soft_scores, target)
    loss_t.backward()
    torch.cuda.synchronize()
    assert float(loss.detach()) == pytest.approx(float(loss_t.detach()), rel=1e-4)
    for name, p in gate.named_parameters():
        ref = p.grad
        err = float((g_hip[name] - ref).abs().max())
        assert err <= 2e-3 * float(ref.abs().max()) + 1e-9, f"{name}: {err:.3e}"
