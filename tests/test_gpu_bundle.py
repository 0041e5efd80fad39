"""Gates of a bundle on the HIP path: ``load_bundle_gates`` onto the GPU in bf16, each layer's
gate run by the HIP kernels with its trained width and its per-head (or scalar) threshold.

The bundle is written in the reference exporter's layout (tasft/bundle/export.py:193-290);
the loader replaces tasft/inference/tasft_model.py:555-580. Logits are compared with the
float64 oracle of the gate formula (tasft/modules/attn_gate.py:241-277) on the loaded
(bf16-rounded) weights; masks must be bit-exact given the kernel's own logits, away from
the threshold, as in the gate tests.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import require_gpu, to_np, write_bundle
from oracle import tasft_oracle as orc
from tasft_amd import workloads as wl
from tasft_amd.inference.bundle_gates import load_bundle_gates
from tasft_amd.modules import AttnGate

pytestmark = pytest.mark.gpu

LOGIT_ATOL = 1e-5
LOGIT_RTOL = 1e-4
TAU_BAND = 1e-6

# (block size, {layer: (hidden width or None for the default, per-head thresholds?)})
BUNDLES = [
    (64, {0: (128, True), 1: (None, False), 5: (48, True)}),
    (32, {2: (64, True)}),
    (128, {0: (None, True)}),
]


@pytest.mark.parametrize(("bs", "layers"), BUNDLES, ids=[f"block{b[0]}" for b in BUNDLES])
def test_bundle_gates_run_on_hip_path(tmp_path, bs, layers):
    dev = require_gpu()
    B, Hq, Hkv, S, D = 2, 8, 2, 1000, 128
    q = wl.randn_bf16((B, Hq, S, D), 7100 + bs, scale=1.0)
    k = wl.randn_bf16((B, Hkv, S, D), 7200 + bs, scale=1.0)
    gates, per_head = {}, {}
    for i, (hidden, ph) in layers.items():
        torch.manual_seed(7300 + 10 * i + bs)
        gates[i] = AttnGate(num_heads=Hq, head_dim=D, block_size=bs, gate_hidden_dim=hidden)
        if ph:
            # Per-head taus near each head's median causal score: dense enough masks, and a
            # different tau per head (the loader must keep the order).
            with torch.no_grad():
                soft = gates[i](q.float(), k.float().repeat_interleave(Hq // Hkv, 1)).soft_scores
            per_head[i] = wl.per_head_threshold(soft.float(), keep_causal=0.3 + 0.05 * (i % 3)).tolist()
    write_bundle(tmp_path, gates, per_head, block_size=bs, scalar_tau=0.5)

    bg = load_bundle_gates(tmp_path, num_heads=Hq, head_dim=D, device=dev, dtype=torch.bfloat16)
    assert sorted(bg.gates) == sorted(layers)
    qd, kd = q.to(dev), k.to(dev)
    for i, (hidden, ph) in layers.items():
        gate = bg.gates[i]
        assert gate.gate_hidden_dim == (hidden if hidden is not None else max(32, D // 4))
        assert gate.block_size == bs and bg.block_sizes[i] == bs
        tau = bg.thresholds[i]
        if ph:
            assert isinstance(tau, torch.Tensor) and tau.device.type == "cuda"
            np.testing.assert_array_equal(tau.cpu().numpy(), np.asarray(per_head[i], np.float32))
        else:
            assert tau == 0.5
        print(f"bundle block {bs} layer {i} hidden {gate.gate_hidden_dim} per-head {ph}", flush=True)
        with torch.no_grad():
            out = gate(qd, kd, threshold=tau, return_logits=True)
        torch.cuda.synchronize()
        # The HIP kernels return fp32 soft scores whatever the module dtype; the torch
        # formula would return the module's bf16.
        assert out.soft_scores.dtype == torch.float32 and out.logits is not None
        w_in = to_np(gate.gate_proj_in.weight)
        b_in = to_np(gate.gate_proj_in.bias)
        w_out = to_np(gate.gate_proj_out.weight)
        ref = orc.gate_logits(to_np(q), to_np(k), w_in, b_in, w_out, bs, dtype=np.float64)
        logits = to_np(out.logits)
        np.testing.assert_allclose(logits, ref, rtol=LOGIT_RTOL, atol=LOGIT_ATOL)
        taus = tau.cpu().numpy() if isinstance(tau, torch.Tensor) else tau
        soft_ref, hard_ref = orc.threshold_mask(logits, taus, True)
        t = np.asarray(taus, dtype=np.float32)
        t = t.reshape(1, -1, 1, 1) if t.ndim == 1 else t
        decisive = np.abs(soft_ref - t) > TAU_BAND
        hard = out.hard_mask.cpu().numpy()
        assert np.array_equal(hard[decisive], hard_ref[decisive]), f"layer {i}: mask differs"
        causal = np.tril(np.ones(hard.shape[-2:], dtype=bool))
        density = hard[..., causal].mean()
        assert 0.02 < density < 0.98, f"layer {i}: degenerate mask (causal density {density:.3f})"
