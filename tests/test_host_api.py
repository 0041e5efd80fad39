"""Host-side API of the drop-in modules (no GPU): constructors, validation, statistics.

Mirrors the reference's CPU unit tests for the same API (tests/unit/test_kernel.py,
tests/unit/test_attn_gate.py, tests/unit/test_edge_cases.py) where they apply.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from helpers import write_bundle
from tasft_amd.exceptions import KernelError, NaNDetectedError, TASFTError, ValidationError
from tasft_amd.kernels import (
    BlockSparseFlashAttention,
    KernelBackend,
    KernelConfig,
    LayerKernelConfig,
    detect_kernels,
)
from tasft_amd.modules import AttnGate, GateOutput
from tasft_amd.training import TASFTObjective


class TestBlockSparseInit:
    def test_invalid_block_size_raises(self):
        with pytest.raises(ValueError, match="block_size"):
            BlockSparseFlashAttention(block_size=16)

    @pytest.mark.parametrize("bs", [32, 64, 128])
    def test_valid_block_sizes(self, bs):
        assert BlockSparseFlashAttention(block_size=bs).block_size == bs

    def test_min_sparsity_range(self):
        with pytest.raises(ValueError, match="min_sparsity_for_speedup"):
            BlockSparseFlashAttention(min_sparsity_for_speedup=1.5)

    def test_auto_selects_hip_backend(self):
        assert BlockSparseFlashAttention().backend == KernelBackend.HIP_GFX950

    @pytest.mark.parametrize("backend", [KernelBackend.TRITON, KernelBackend.FLASH_ATTN_SPARSE])
    def test_unavailable_backend_raises(self, backend):
        with pytest.raises(KernelError, match="not available"):
            BlockSparseFlashAttention(backend=backend)

    def test_detect_kernels_dense_fallback_last(self):
        avail = detect_kernels()
        assert avail[-1] == KernelBackend.DENSE_FALLBACK
        assert KernelBackend.HIP_GFX950 in avail  # the library is built in-tree

    def test_sparsity_stats(self):
        bsfa = BlockSparseFlashAttention(block_size=64)
        mask = torch.zeros(1, 4, 8, 8, dtype=torch.bool)
        mask[:, :, :4, :] = True
        st = bsfa.compute_sparsity_stats(mask)
        assert (st.total_blocks, st.active_blocks) == (256, 128)
        assert st.sparsity_ratio == pytest.approx(0.5)
        assert st.estimated_speedup == pytest.approx(1.0 / (1.0 - 0.5 * 0.98))

    def test_speedup_model(self):
        assert abs(BlockSparseFlashAttention.estimate_speedup(0.0) - 1.0) < 0.05
        assert BlockSparseFlashAttention.estimate_speedup(0.9) > 3.0
        prev = 0.0
        for pct in range(0, 100, 5):
            s = BlockSparseFlashAttention.estimate_speedup(pct / 100)
            assert s >= prev
            prev = s


class TestBlockSparseValidation:
    def _bsfa(self):
        return BlockSparseFlashAttention(block_size=32, min_sparsity_for_speedup=0.0)

    def test_ndim(self):
        x = torch.zeros(2, 64, 32)
        with pytest.raises(KernelError, match="Expected 4D tensors"):
            self._bsfa().forward(x, x, x, torch.ones(1, 1, 2, 2, dtype=torch.bool))

    def test_shape_mismatch(self):
        q = torch.zeros(1, 4, 64, 32)
        k = torch.zeros(1, 3, 64, 32)  # 4 % 3 != 0: not a GQA layout
        with pytest.raises(KernelError, match="Q, K, V shapes must match"):
            self._bsfa().forward(q, k, k, torch.ones(1, 4, 2, 2, dtype=torch.bool))

    def test_cpu_tensors_rejected(self):
        q = torch.zeros(1, 4, 64, 32)
        kv = torch.zeros(1, 2, 64, 32)  # GQA layout passes the shape check
        with pytest.raises(KernelError, match="Tensors must be on CUDA device"):
            self._bsfa().forward(q, kv, kv, torch.ones(1, 4, 2, 2, dtype=torch.bool))

    def test_decode_shape_checks(self):
        q = torch.zeros(1, 4, 2, 32)
        kv = torch.zeros(1, 2, 64, 32)
        with pytest.raises(KernelError, match=r"\[B, H, 1, D\]"):
            self._bsfa().forward_decode(q, kv, kv, torch.ones(1, 4, 1, 2, dtype=torch.bool))


class TestKernelConfig:
    def test_defaults_and_lookup(self):
        lc = LayerKernelConfig(layer_idx=3, threshold_tau=0.7, target_sparsity=0.8,
                               achieved_sparsity_validation=0.79)
        kc = KernelConfig(per_layer_config={3: lc})
        assert kc.get_layer_threshold(3) == 0.7
        assert kc.get_layer_threshold(0) == 0.5
        assert kc.get_layer_block_size(3) == 64

    def test_validation(self):
        with pytest.raises(ValueError, match="threshold_tau"):
            LayerKernelConfig(layer_idx=0, threshold_tau=1.0, target_sparsity=0.5,
                              achieved_sparsity_validation=0.5)
        with pytest.raises(ValueError, match="block_size"):
            KernelConfig(block_size=48)
        lc = LayerKernelConfig(layer_idx=1, threshold_tau=0.5, target_sparsity=0.5,
                               achieved_sparsity_validation=0.5)
        with pytest.raises(ValueError, match="doesn't match"):
            KernelConfig(per_layer_config={2: lc})
        with pytest.raises(ValueError):
            KernelConfig(unknown_field=1)


class TestAttnGateHost:
    def test_defaults(self):
        g = AttnGate(num_heads=4, head_dim=32)
        assert (g.block_size, g.default_threshold, g.gate_hidden_dim) == (64, 0.5, 32)
        assert AttnGate(num_heads=4, head_dim=256).gate_hidden_dim == 64

    @pytest.mark.parametrize(("kwargs", "msg"), [
        ({"num_heads": 0, "head_dim": 32}, "num_heads must be positive"),
        ({"num_heads": 4, "head_dim": 0}, "head_dim must be positive"),
        ({"num_heads": 4, "head_dim": 32, "block_size": 0}, "block_size must be positive"),
        ({"num_heads": 4, "head_dim": 32, "default_threshold": 1.5}, "default_threshold must be in"),
    ])
    def test_constructor_errors(self, kwargs, msg):
        with pytest.raises(ValidationError, match=msg):
            AttnGate(**kwargs)

    def test_state_dict_keys_and_param_count(self):
        g = AttnGate(num_heads=32, head_dim=128, gate_hidden_dim=128)
        assert set(g.state_dict()) == {"gate_proj_in.weight", "gate_proj_in.bias", "gate_proj_out.weight"}
        assert g.num_parameters == 256 * 128 + 128 + 128
        r = g.extra_repr()
        assert "num_heads=32" in r and "head_dim=128" in r and "block_size=64" in r

    def test_seeded_init_matches_reference_order(self):
        """Same RNG consumption as the reference: Linear default init, then xavier/zeros/normal."""
        torch.manual_seed(0)
        g = AttnGate(num_heads=2, head_dim=16, gate_hidden_dim=8)
        torch.manual_seed(0)
        a = torch.nn.Linear(32, 8)
        b = torch.nn.Linear(8, 1, bias=False)
        torch.nn.init.xavier_uniform_(a.weight)
        torch.nn.init.zeros_(a.bias)
        torch.nn.init.normal_(b.weight, std=0.01)
        assert torch.equal(g.gate_proj_in.weight, a.weight)
        assert torch.equal(g.gate_proj_out.weight, b.weight)

    @pytest.mark.parametrize(("q", "k", "msg"), [
        ((4, 64, 32), (1, 4, 64, 32), "Expected 4D Q tensor"),
        ((1, 4, 64, 32), (4, 64, 32), "Expected 4D K tensor"),
        ((1, 4, 64, 32), (1, 4, 128, 32), "Q and K must have same shape"),
        ((1, 8, 64, 32), (1, 8, 64, 32), "Expected 4 heads"),
        ((1, 4, 64, 64), (1, 4, 64, 64), "Expected head_dim=32"),
        ((1, 4, 0, 32), (1, 4, 0, 32), "Sequence length must be > 0"),
    ])
    def test_forward_validation_messages(self, q, k, msg):
        g = AttnGate(num_heads=4, head_dim=32, block_size=8)
        with pytest.raises(ValidationError, match=msg):
            g(torch.randn(q), torch.randn(k))

    def test_cpu_fp32_matches_reference_concat_formula(self):
        """CPU fp32 runs the reference formula: logits equal the materialised-concat
        Linear-ReLU-Linear of the oracle (attn_gate.py:248-257), masks follow from them."""
        from oracle import tasft_oracle as orc

        torch.manual_seed(3)
        g = AttnGate(num_heads=4, head_dim=32, block_size=8)
        q, k = torch.randn(2, 4, 60, 32), torch.randn(2, 4, 60, 32)
        out = g(q, k, threshold=0.5, return_logits=True)
        w_in, b_in = g.gate_proj_in.weight.detach().numpy(), g.gate_proj_in.bias.detach().numpy()
        w_out = g.gate_proj_out.weight.detach().numpy()
        qb = orc.pool_to_blocks(q.double().numpy(), 8)
        kb = orc.pool_to_blocks(k.double().numpy(), 8)
        ref = orc.gate_logits_concat(qb, kb, w_in.astype(np.float64), b_in.astype(np.float64),
                                     w_out.astype(np.float64))
        np.testing.assert_allclose(out.logits.detach().numpy(), ref, rtol=1e-5, atol=1e-6)
        assert out.soft_scores.dtype == torch.float32
        soft = out.soft_scores.detach()
        assert (soft[..., torch.ones(8, 8, dtype=torch.bool).triu(1)] == 0).all()
        assert torch.equal(out.hard_mask, soft >= 0.5)
        assert out.sparsity_ratio == pytest.approx(1.0 - out.hard_mask.float().mean().item())

    # The shapes, ranges and edge cases of the reference's own CPU tests
    # (tests/unit/test_attn_gate.py:123-141, 160-236, 244-278, 289-318).
    @pytest.mark.parametrize(("B", "H", "S", "D", "bs"), [
        (1, 4, 64, 32, 8), (2, 8, 128, 64, 16), (4, 16, 256, 128, 32), (1, 32, 2048, 128, 64)])
    def test_cpu_output_shapes(self, B, H, S, D, bs):
        g = AttnGate(num_heads=H, head_dim=D, block_size=bs)
        out = g(torch.randn(B, H, S, D), torch.randn(B, H, S, D))
        nb = (S + bs - 1) // bs
        assert isinstance(out, GateOutput)
        assert out.soft_scores.shape == (B, H, nb, nb) and out.hard_mask.shape == (B, H, nb, nb)
        assert out.hard_mask.dtype == torch.bool
        assert (out.num_blocks_q, out.num_blocks_k) == (nb, nb)

    @pytest.mark.parametrize("scale", [1.0, 1000.0, 0.0])
    def test_cpu_scores_in_unit_interval(self, scale):
        g = AttnGate(num_heads=4, head_dim=32, block_size=8)
        out = g(torch.randn(2, 4, 64, 32) * scale, torch.randn(2, 4, 64, 32) * scale)
        s = out.soft_scores
        assert not s.isnan().any() and not s.isinf().any()
        assert s.min() >= 0.0 and s.max() <= 1.0

    def test_cpu_sparsity_edges_and_compute_sparsity(self):
        g = AttnGate(num_heads=4, head_dim=32, block_size=8)
        q, k = torch.randn(1, 4, 64, 32), torch.randn(1, 4, 64, 32)
        out0 = g(q, k, threshold=0.0)
        assert out0.sparsity_ratio == pytest.approx(0.0, abs=1e-6) and out0.hard_mask.all()
        out1 = g(q, k, threshold=1.0 + 1e-6)
        assert out1.sparsity_ratio == pytest.approx(1.0, abs=1e-6) and not out1.hard_mask.any()
        out = g(q, k, threshold=0.5)
        assert g.compute_sparsity(out.soft_scores, 0.5) == pytest.approx(out.sparsity_ratio, abs=1e-6)

    def test_cpu_bf16_and_fp16_modules(self):
        for dt in (torch.bfloat16, torch.float16):
            g = AttnGate(num_heads=8, head_dim=64, block_size=16).to(dt)
            out = g(torch.randn(2, 8, 256, 64, dtype=dt), torch.randn(2, 8, 256, 64, dtype=dt))
            assert out.soft_scores.dtype == dt  # the module dtype, as the reference returns
            assert not out.soft_scores.isnan().any() and not out.soft_scores.isinf().any()
            assert out.soft_scores.min() >= 0.0 and out.soft_scores.max() <= 1.0
        g32 = AttnGate(num_heads=4, head_dim=32, block_size=8)
        g16 = AttnGate(num_heads=4, head_dim=32, block_size=8).to(torch.bfloat16)
        q = torch.randn(1, 4, 64, 32)
        assert g32(q, q).soft_scores.shape == g16(q.bfloat16(), q.bfloat16()).soft_scores.shape

    @pytest.mark.parametrize(("S", "bs"), [(65, 64), (100, 64), (127, 64), (33, 16), (1, 8), (7, 8), (9, 8)])
    def test_cpu_non_divisible_seq_len(self, S, bs):
        g = AttnGate(num_heads=4, head_dim=32, block_size=bs)
        out = g(torch.randn(1, 4, S, 32), torch.randn(1, 4, S, 32))
        nb = (S + bs - 1) // bs
        assert out.num_blocks_q == nb and out.soft_scores.shape == (1, 4, nb, nb)

    def test_cpu_gqa_and_per_head_threshold(self):
        g = AttnGate(num_heads=8, head_dim=32, block_size=8)
        q, k = torch.randn(1, 8, 64, 32), torch.randn(1, 2, 64, 32)
        a = g(q, k, threshold=torch.full((8,), 0.5))
        b = g(q, k.repeat_interleave(4, dim=1), threshold=0.5)
        torch.testing.assert_close(a.soft_scores, b.soft_scores)
        assert torch.equal(a.hard_mask, b.hard_mask)

    def test_cached_decoding_rejected_without_query_offset(self):
        """S_q != S_k raises as the reference does (pinned by its
        tests/integration/test_model_families.py:915-948)."""
        g = AttnGate(num_heads=4, head_dim=16, block_size=32)
        with pytest.raises(ValidationError, match="Q and K must have same shape"):
            g(torch.randn(1, 4, 8, 16), torch.randn(1, 4, 24, 16))

    @pytest.mark.parametrize("t", [44, 40, 32, 0])
    def test_query_offset_row_equals_full_gate_row(self, t):
        """query_offset = t with the block's earlier queries as q_block_sum gives exactly
        the row t // block of the gate on tokens 0 .. t."""
        torch.manual_seed(1)
        g = AttnGate(num_heads=4, head_dim=32, block_size=8)
        q, k = torch.randn(2, 4, 45, 32), torch.randn(2, 2, 45, 32)
        r = t // 8
        row = g(q[:, :, t:t + 1], k[:, :, :t + 1], return_logits=True, query_offset=t,
                q_block_sum=q[:, :, r * 8:t].sum(2))
        full = g(q[:, :, :t + 1], k[:, :, :t + 1], return_logits=True)
        assert row.soft_scores.shape == (2, 4, 1, r + 1)
        torch.testing.assert_close(row.logits[:, :, 0], full.logits[:, :, r], rtol=0, atol=1e-6)
        assert torch.equal(row.hard_mask[:, :, 0], full.hard_mask[:, :, r])
        chunk = g(q[:, :, 16:45], k, return_logits=True, query_offset=16)
        torch.testing.assert_close(chunk.logits, g(q, k, return_logits=True).logits[:, :, 2:], rtol=0, atol=1e-6)

    def test_cpu_gradients_reach_gate_parameters(self):
        g = AttnGate(num_heads=4, head_dim=32, block_size=8)
        out = g(torch.randn(1, 4, 64, 32), torch.randn(1, 4, 64, 32))
        out.soft_scores.sum().backward()
        for name, p in g.named_parameters():
            assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().sum() > 0, name

    def test_gate_output_frozen_and_lazy(self):
        out = GateOutput(soft_scores=torch.zeros(1, 1, 2, 2), hard_mask=torch.zeros(1, 1, 2, 2, dtype=torch.bool),
                         num_blocks_q=2, num_blocks_k=2, active_count=torch.tensor([1]))
        assert out.sparsity_ratio == pytest.approx(0.75)
        with pytest.raises(AttributeError):
            out.sparsity_ratio = 0.5
        with pytest.raises(dataclasses.FrozenInstanceError):
            out.hard_mask = None


class TestGateTargetDense:
    def test_reference_dense_path_on_scores(self):
        attn = torch.arange(1, 17, dtype=torch.float32).reshape(1, 1, 4, 4)
        t = TASFTObjective.compute_gate_target(attn, block_size=2)
        ref = torch.softmax(torch.tensor([6.0, 8.0, 14.0, 16.0]), 0).reshape(1, 1, 2, 2)
        torch.testing.assert_close(t, ref)

    def test_nan_raises_with_context(self):
        attn = torch.tensor([[[[float("nan"), 1.0], [1.0, 1.0]]]])
        with pytest.raises(NaNDetectedError) as ei:
            TASFTObjective.compute_gate_target(attn, block_size=1)
        assert ei.value.context["has_nan"] is True
        assert isinstance(ei.value, TASFTError)

    def test_block_size_zero(self):
        with pytest.raises(ValueError, match="block_size must be > 0"):
            TASFTObjective.compute_gate_target(torch.randn(1, 1, 4, 4), block_size=0)


# ----------------------------------------------------------------------------- decode splits
def test_default_decode_splits_fill_the_resident_workgroups_once():
    from tasft_amd.kernels import default_decode_splits

    # About one workgroup per CU (256), whatever the head count.
    assert default_decode_splits(64, 8, 512) == 1          # config 3 (512 workgroups)
    assert default_decode_splits(64, 4, 512, 4) == 1
    assert default_decode_splits(4, 8, 64) == 8
    assert default_decode_splits(64, 4, 512, 7) == 1       # Qwen-2.5-7B at config-3 batch
    assert default_decode_splits(8, 4, 512, 7) == 8
    assert default_decode_splits(4, 8, 64, 16) == 8
    # Never fewer splits than keep each within 1024 key blocks, never more than blocks // 4.
    assert default_decode_splits(64, 8, 5000) == 5
    assert default_decode_splits(1, 1, 8, 7) == 2


# ----------------------------------------------------------------------------- varlen validation
def _varlen_args(T=40, H=4, Hkv=2, D=64):
    q = torch.zeros(T, H, D, dtype=torch.bfloat16)
    k = torch.zeros(T, Hkv, D, dtype=torch.bfloat16)
    return q, k, k.clone()


def test_forward_varlen_validates_before_any_launch():
    bsfa = BlockSparseFlashAttention(block_size=32, min_sparsity_for_speedup=0.0)
    q, k, v = _varlen_args()
    mask = torch.ones(2, 4, 1, 1, dtype=torch.bool)
    with pytest.raises(KernelError, match=r"packed q, k, v of shape \[T, H, D\]"):
        bsfa.forward_varlen(q[None], k, v, mask, torch.tensor([0, 10, 30], dtype=torch.int32))
    with pytest.raises(KernelError, match="Hq % Hkv == 0"):
        bsfa.forward_varlen(q, k[:, :1].expand(40, 3, 64), v, mask, torch.tensor([0, 10, 30]))
    with pytest.raises(KernelError, match="start at 0"):
        bsfa.forward_varlen(q, k, v, mask, torch.tensor([1, 10, 30], dtype=torch.int32))
    with pytest.raises(KernelError, match="non-decreasing"):
        bsfa.forward_varlen(q, k, v, mask, torch.tensor([0, 20, 10], dtype=torch.int32))
    with pytest.raises(KernelError, match="end at <= T"):
        bsfa.forward_varlen(q, k, v, mask, torch.tensor([0, 20, 41], dtype=torch.int32))
    with pytest.raises(KernelError, match="more than max_seqlen"):
        bsfa.forward_varlen(q, k, v, mask, torch.tensor([0, 10, 30], dtype=torch.int32), 16)
    with pytest.raises(KernelError, match="block_mask shape mismatch"):
        bsfa.forward_varlen(q, k, v, torch.ones(2, 4, 2, 2, dtype=torch.bool),
                            torch.tensor([0, 10, 30], dtype=torch.int32))
    with pytest.raises(KernelError, match="head_dim"):
        q2, k2, v2 = _varlen_args(D=32)
        bsfa.forward_varlen(q2, k2, v2, mask, torch.tensor([0, 10, 30], dtype=torch.int32))
    # valid arguments on CPU tensors stop at the device check, before the library
    with pytest.raises(KernelError, match="same GPU device"):
        bsfa.forward_varlen(q, k, v, mask, torch.tensor([0, 10, 30], dtype=torch.int32))


# ----------------------------------------------------------------------------- kernel_config.json
def test_kernel_config_loads_reference_and_exporter_files_and_per_head_thresholds():
    import json

    from tasft_amd.kernels import KernelConfig

    # A file in the reference loader's format loads unchanged.
    ref = {"block_size": 64, "global_threshold": 0.5, "min_sparsity_for_speedup": 0.5,
           "per_layer_config": {"0": {"layer_idx": 0, "threshold_tau": 0.4, "target_sparsity": 0.8,
                                      "achieved_sparsity_validation": 0.79}}}
    cfg = KernelConfig.model_validate(ref)
    assert cfg.get_layer_threshold(0) == 0.4 and cfg.get_layer_threshold(3) == 0.5
    assert cfg.get_layer_head_thresholds(0, 4) == (0.4, 0.4, 0.4, 0.4)
    # The exporter's per-layer record (with gate_loss_validation) loads too.
    exp = json.loads(json.dumps(ref))
    exp["per_layer_config"]["0"]["gate_loss_validation"] = 0.031
    assert KernelConfig.model_validate(exp).per_layer_config[0].gate_loss_validation == 0.031
    # Per-head thresholds and the gate width round-trip through JSON.
    ph = json.loads(json.dumps(ref))
    ph["per_layer_config"]["0"].update(threshold_tau_per_head=[0.3, 0.4, 0.5, 0.6], gate_hidden_dim=32)
    cfg2 = KernelConfig.model_validate_json(KernelConfig.model_validate(ph).model_dump_json())
    assert cfg2.get_layer_head_thresholds(0, 4) == (0.3, 0.4, 0.5, 0.6)
    assert cfg2.per_layer_config[0].gate_hidden_dim == 32
    with pytest.raises(ValueError, match="expected 8"):
        cfg2.get_layer_head_thresholds(0, 8)
    bad = json.loads(json.dumps(ph))
    bad["per_layer_config"]["0"]["threshold_tau_per_head"] = [0.3, 1.0]
    with pytest.raises(ValueError, match=r"threshold_tau_per_head\[1\] must be in \(0, 1\)"):
        KernelConfig.model_validate(bad)
    unknown = json.loads(json.dumps(ref))
    unknown["per_layer_config"]["0"]["surprise"] = 1
    with pytest.raises(ValueError):
        KernelConfig.model_validate(unknown)


# ----------------------------------------------------------------------------- bundle gates
def test_bundle_gates_keep_trained_width_and_per_head_thresholds(tmp_path):
    from tasft_amd.exceptions import BundleError, ChecksumError
    from tasft_amd.inference.bundle_gates import load_bundle_gates

    torch.manual_seed(4)
    gates = {0: AttnGate(num_heads=4, head_dim=32, gate_hidden_dim=48),   # non-default width
             1: AttnGate(num_heads=4, head_dim=32)}                       # default width (32)
    per_head = {0: [0.3, 0.4, 0.5, 0.6]}
    write_bundle(tmp_path, gates, per_head)
    bg = load_bundle_gates(tmp_path, num_heads=4, head_dim=32)
    assert sorted(bg.gates) == [0, 1]
    assert bg.gates[0].gate_hidden_dim == 48 and bg.gates[1].gate_hidden_dim == 32
    assert torch.equal(bg.thresholds[0], torch.tensor(per_head[0]))
    assert bg.thresholds[1] == 0.5
    q, k = torch.randn(1, 4, 256, 32), torch.randn(1, 4, 256, 32)
    for i in (0, 1):
        a = bg.gates[i](q, k, threshold=bg.thresholds[i], return_logits=True)
        b = gates[i](q, k, threshold=bg.thresholds[i], return_logits=True)
        torch.testing.assert_close(a.logits, b.logits, rtol=0, atol=0)
        assert torch.equal(a.hard_mask, b.hard_mask)
    # The reference loader's default-width construction cannot hold layer 0's state.
    with pytest.raises(RuntimeError, match="size mismatch"):
        AttnGate(num_heads=4, head_dim=32).load_state_dict(gates[0].state_dict())
    # A tampered gate file fails its checksum; a wrong head_dim fails the shape check.
    (tmp_path / "gates" / "layer_1_gate.safetensors").write_bytes(b"x")
    with pytest.raises(ChecksumError):
        load_bundle_gates(tmp_path, num_heads=4, head_dim=32)
    (tmp_path / "b2").mkdir()
    write_bundle(tmp_path / "b2", {0: gates[0]}, {})
    with pytest.raises(BundleError, match="head_dim=64"):
        load_bundle_gates(tmp_path / "b2", num_heads=4, head_dim=64)


@pytest.mark.parametrize("K", [100, 256, 512, 4096 + 256])
def test_gate_weight_grad_split_over_k_equals_one_product(K):
    """The gate backward's d^T @ m, summed over K chunks as a batched product (K a multiple
    of the chunk, at least two chunks) or taken as one product (otherwise)."""
    from tasft_amd.modules.attn_gate import _weight_grad

    g = torch.Generator().manual_seed(K)
    d = torch.randn(K, 48, generator=g, dtype=torch.float64)
    m = torch.randn(K, 80, generator=g, dtype=torch.float64)
    got = _weight_grad(d, m)
    assert got.shape == (48, 80)
    torch.testing.assert_close(got, d.t() @ m, rtol=1e-12, atol=1e-10)
