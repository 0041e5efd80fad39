"""HIP-graph capture of the hot path: the gate (one kernel after its counter reset), the
prefill (two-wave kernel; the persistent four-wave kernel with its ticket reset; block 128 on
the block-64 kernel) and the split-K decode are captured once and replayed with new inputs.

Each replay is preceded by eager work on the same tensors (the same call run eagerly on the
replay's inputs, then a synchronisation), and every replay must equal that eager result bit
for bit: counters, tickets and workspaces that a replay finds must have been reset by kernels
inside the graph, since no host code runs between replays.
"""
from __future__ import annotations

import pytest
import torch

from helpers import require_gpu
from tasft_amd import workloads as wl
from tasft_amd.kernels import BlockSparseFlashAttention
from tasft_amd.modules import AttnGate

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _capture(fn):
    """Warm ``fn`` up on a side stream, then capture one call; returns (graph, outputs)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def test_gate_one_kernel_replays():
    dev = require_gpu()
    B, Hq, Hkv, S, D, hidden = 2, 8, 2, 2048, 128, 64
    torch.manual_seed(3)
    gate = AttnGate(num_heads=Hq, head_dim=D, block_size=64, gate_hidden_dim=hidden).to(dev)
    gate.requires_grad_(False)
    taus = torch.linspace(0.45, 0.55, Hq, device=dev)
    q = wl.randn_bf16((B, Hq, S, D), 1, scale=1.0).to(dev)
    k = wl.randn_bf16((B, Hkv, S, D), 2, scale=1.0).to(dev)

    def run():
        with torch.no_grad():
            o = gate(q, k, threshold=taus, force_diagonal=True)
        return o.soft_scores, o.hard_mask, o._active

    g, (soft, mask, active) = _capture(run)
    for r in range(REPLAYS):
        q.copy_(wl.randn_bf16((B, Hq, S, D), 10 + r, scale=1.0).to(dev))
        k.copy_(wl.randn_bf16((B, Hkv, S, D), 20 + r, scale=1.0).to(dev))
        ref_soft, ref_mask, ref_active = (t.clone() for t in run())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(soft, ref_soft), f"replay {r}: soft scores"
        assert torch.equal(mask, ref_mask), f"replay {r}: mask"
        assert int(active.item()) == int(ref_active.item()) == int(ref_mask.sum().item())


@pytest.mark.parametrize(("D", "bs"), [(128, 64), (64, 64), (128, 128)])
def test_prefill_replays(D, bs):
    dev = require_gpu()
    B, Hq, Hkv, S = 1, 8, 2, 1536
    bsfa = BlockSparseFlashAttention(block_size=bs, min_sparsity_for_speedup=0.0)
    q = wl.randn_bf16((B, Hq, S, D), 31, scale=1.0).to(dev)
    k = wl.randn_bf16((B, Hkv, S, D), 32, scale=1.0).to(dev)
    v = wl.randn_bf16((B, Hkv, S, D), 33, scale=1.0).to(dev)
    shape = wl.Shape(B, Hq, Hkv, S, D, bs)
    mask = wl.bernoulli_causal_mask(shape, 0.4, 34).to(dev)

    def run():
        with torch.no_grad():
            return bsfa.forward(q, k, v, mask, causal=True)

    g, out = _capture(run)
    for r in range(REPLAYS):
        q.copy_(wl.randn_bf16((B, Hq, S, D), 40 + r, scale=1.0).to(dev))
        v.copy_(wl.randn_bf16((B, Hkv, S, D), 50 + r, scale=1.0).to(dev))
        mask.copy_(wl.bernoulli_causal_mask(shape, 0.3 + 0.1 * r, 60 + r).to(dev))
        ref = run().clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r}"


def test_decode_replays():
    dev = require_gpu()
    B, Hq, Hkv, S, D = 4, 8, 2, 4096, 128
    nb = S // 64
    bsfa = BlockSparseFlashAttention(block_size=64, min_sparsity_for_speedup=0.0)
    q = wl.randn_bf16((B, Hq, 1, D), 71, scale=1.0).to(dev)
    kc = wl.randn_bf16((B, Hkv, S, D), 72, scale=1.0).to(dev)
    vc = wl.randn_bf16((B, Hkv, S, D), 73, scale=1.0).to(dev)
    mask = (torch.rand((B, Hq, 1, nb), generator=torch.Generator().manual_seed(74)) < 0.2).to(dev)
    mask[..., -1] = True
    lens = torch.full((B,), S, dtype=torch.int32, device=dev)

    def run():
        with torch.no_grad():
            return bsfa.forward_decode(q, kc, vc, mask, kv_lens=lens, num_splits=4)

    g, out = _capture(run)
    for r in range(REPLAYS):
        q.copy_(wl.randn_bf16((B, Hq, 1, D), 80 + r, scale=1.0).to(dev))
        lens.copy_(torch.tensor([S - 100 * r - b for b in range(B)], dtype=torch.int32))
        ref = run().clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r}"
