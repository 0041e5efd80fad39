"""Cached decode steps through the gate-driven wiring (``SparseAttentionDecoder``).

Each step's block selection must equal the oracle gate's row for the new token's query
block on the whole sequence so far (soft scores within fp32 rounding, masks bit-exact away
from tau, the diagonal forced on), and the step's output must match the oracle's sparse
decode under that selection, with K/V in their GQA layout (Hkv heads).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, require_gpu, to_np
from oracle import tasft_oracle as orc
from tasft_amd import workloads as wl
from tasft_amd.inference import SparseAttentionDecoder
from tasft_amd.modules import AttnGate

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(("B", "Hq", "Hkv", "D", "hid", "S0", "steps"), [
    (2, 8, 2, 128, 64, 1021, 5),    # crosses the block boundary at 1024
    (1, 4, 4, 64, 32, 128, 3),      # prompt of whole blocks, MHA, D=64
    (1, 16, 2, 128, 128, 2045, 4),  # 8 query heads per KV head (one launch per step), boundary
    (1, 8, 2, 64, 64, 8250, 2),     # 130 key blocks: one thread per block in the row kernel
    (2, 8, 1, 64, 320, 190, 3),     # hidden 320 (> 256): torch state update +
                                    # tasft_gate_rows_fwd
])
def test_cached_decode_steps_match_oracle(B, Hq, Hkv, D, hid, S0, steps, dtype=torch.bfloat16):
    dev = require_gpu()
    bs = 64
    n = S0 + steps
    q = wl.randn_bf16((B, Hq, n, D), 71 + n, scale=1.0).to(dtype)
    k = wl.randn_bf16((B, Hkv, n, D), 72 + n, scale=1.0).to(dtype)
    v = wl.randn_bf16((B, Hkv, n, D), 73 + n, scale=1.0).to(dtype)
    torch.manual_seed(n)
    gate = AttnGate(num_heads=Hq, head_dim=D, block_size=bs, gate_hidden_dim=hid).to(dev).requires_grad_(False)
    tau = 0.5
    dec = SparseAttentionDecoder(gate, tau, max_len=max(4096, n))
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out_p, g_p = dec.prefill(qd[:, :, :S0], kd[:, :, :S0], vd[:, :, :S0])
    w_in = gate.gate_proj_in.weight.cpu().numpy()
    b_in = gate.gate_proj_in.bias.cpu().numpy()
    w_out = gate.gate_proj_out.weight.cpu().numpy()
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    for t in range(S0, n):
        print(f"decode step t={t}", flush=True)
        out, row = dec.step(qd[:, :, t:t + 1], kd[:, :, :t + 1], vd[:, :, :t + 1])
        torch.cuda.synchronize()
        i = t // bs
        logits = orc.gate_logits(qn[:, :, :t + 1], kn[:, :, :t + 1], w_in, b_in, w_out, bs,
                                 dtype=np.float64)[:, :, i]
        soft_ref = 1.0 / (1.0 + np.exp(-logits))
        soft_ref[..., i + 1:] = 0.0
        soft = to_np(row.soft_scores)[:, :, 0]
        np.testing.assert_allclose(soft, soft_ref, rtol=0, atol=2e-6)
        hard = row.hard_mask.cpu().numpy()[:, :, 0]
        hard_ref = soft_ref >= tau
        hard_ref[..., i] = True  # force_diagonal
        decisive = np.abs(soft_ref - tau) > 1e-6
        decisive[..., i] = True
        assert np.array_equal(hard[decisive], hard_ref[decisive])
        ref = orc.sparse_decode(qn[:, :, t:t + 1], kn[:, :, :t + 1], vn[:, :, :t + 1],
                                row.hard_mask.cpu().numpy(), bs)
        assert_close_bf16(out, ref, f"decode step {t}")
    assert dec.length == n


def test_cached_decode_steps_fp16():
    """fp16 prompt and cache (the same values as a bf16 draw, exact in fp16 at this scale):
    the one-launch rows and the decode run their fp16 instantiations."""
    test_cached_decode_steps_match_oracle(1, 8, 2, 128, 64, 509, 4, dtype=torch.float16)
