"""Pins the CPU oracle against the reference's known answers, library routines and brute force.

None of these checks retypes the oracle's own formula: each compares it with literal
vectors from the reference tests (tests/golden/reference_vectors.json), with a torch
library routine, with an independent pure-Python loop, or with a second formulation.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import tasft_oracle as orc

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


# ----------------------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("case", ["pool_block4", "pool_padding", "pool_single_block"])
def test_pool_matches_reference_vectors(case):
    c = GOLDEN[case]
    got = orc.pool_to_blocks(np.array(c["x"], dtype=np.float32), c["block_size"])
    np.testing.assert_allclose(got, np.array(c["expected"]), atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("case", ["gate_target_4x4", "gate_target_8x8", "gate_target_uniform"])
def test_gate_target_matches_reference_vectors(case):
    c = GOLDEN[case]
    got = orc.gate_target_from_scores(np.array(c["scores"], dtype=np.float64), c["block_size"])
    np.testing.assert_allclose(got, np.array(c["expected"]), atol=1e-6, rtol=1e-6)
    assert got.sum() == pytest.approx(1.0, abs=1e-9)


def test_gate_target_rejects_nan_and_pos_inf_allows_neg_inf():
    x = np.zeros((1, 1, 4, 4))
    x[0, 0, 0, 1] = np.nan
    with pytest.raises(ValueError):
        orc.gate_target_from_scores(x, 2)
    x[0, 0, 0, 1] = np.inf
    with pytest.raises(ValueError):
        orc.gate_target_from_scores(x, 2)
    # Causal -inf (test_numerical_correctness.py:173-184) is allowed and gives a distribution.
    y = np.random.default_rng(0).standard_normal((1, 1, 8, 8))
    y[0, 0][np.triu(np.ones((8, 8), bool), 1)] = -np.inf
    t = orc.gate_target_from_scores(y, 4)
    assert np.isfinite(t).all() and t.sum() == pytest.approx(1.0)


def test_gate_target_matches_torch_maxpool_softmax():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, 37, 37))  # ragged: pads to 40 with -inf
    got = orc.gate_target_from_scores(x, 8)
    t = torch.from_numpy(x)
    t = F.pad(t, (0, 3, 0, 3), value=-math.inf)
    pooled = F.max_pool2d(t, 8, 8)
    ref = F.softmax(pooled.reshape(2, 3, -1), dim=-1).reshape(pooled.shape).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-15)


def test_stats_and_speedup_match_reference_vectors():
    c = GOLDEN["sparsity_stats"]
    m = np.zeros(c["mask_shape"], dtype=bool)
    m[:, :, : c["active_rows"], :] = True
    assert orc.sparsity_stats(m) == (c["total"], c["active"], c["sparsity"])
    for s, v in GOLDEN["speedup"]["points"]:
        assert orc.estimate_speedup(s) == pytest.approx(v, rel=1e-12)
    lo, hi = GOLDEN["speedup"]["bounds"]["at_0"]
    assert lo <= orc.estimate_speedup(0.0) <= hi
    assert orc.estimate_speedup(0.9) > GOLDEN["speedup"]["bounds"]["at_0.9_min"]


# ----------------------------------------------------------------------------- gate
def _torch_gate_reference(q, k, lin_in, lin_out, bs):
    """Gate logits through torch.nn.Linear / relu on the materialised concat."""
    qt, kt = torch.from_numpy(q).float(), torch.from_numpy(k).float()
    B, H, S, D = qt.shape
    pad = (bs - S % bs) % bs
    qt, kt = F.pad(qt, (0, 0, 0, pad)), F.pad(kt, (0, 0, 0, pad))
    nb = qt.shape[2] // bs
    qb = qt.view(B, H, nb, bs, D).mean(3)
    kb = kt.view(B, H, nb, bs, D).mean(3)
    cat = torch.cat([qb.unsqueeze(3).expand(B, H, nb, nb, D), kb.unsqueeze(2).expand(B, H, nb, nb, D)], -1)
    with torch.no_grad():
        return lin_out(F.relu(lin_in(cat))).squeeze(-1).numpy()


def test_gate_logits_match_torch_linear_and_concat_form():
    torch.manual_seed(3)
    D, hid, bs = 16, 24, 8
    lin_in = torch.nn.Linear(2 * D, hid)
    lin_out = torch.nn.Linear(hid, 1, bias=False)
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 4, 30, D)).astype(np.float32)
    k = rng.standard_normal((2, 4, 30, D)).astype(np.float32)
    w_in, b_in = lin_in.weight.detach().numpy(), lin_in.bias.detach().numpy()
    w_out = lin_out.weight.detach().numpy()
    ref = _torch_gate_reference(q, k, lin_in, lin_out, bs)
    dec = orc.gate_logits(q, k, w_in, b_in, w_out, bs, dtype=np.float64)
    cat = orc.gate_logits_concat(orc.pool_to_blocks(q, bs), orc.pool_to_blocks(k, bs), w_in, b_in, w_out)
    np.testing.assert_allclose(dec, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(cat, ref, rtol=1e-5, atol=1e-6)


def test_gate_logits_gqa_equals_expanded_k():
    rng = np.random.default_rng(4)
    D, hid, bs = 16, 32, 4
    w_in = rng.standard_normal((hid, 2 * D)).astype(np.float32)
    b_in = rng.standard_normal(hid).astype(np.float32)
    w_out = rng.standard_normal((1, hid)).astype(np.float32)
    q = rng.standard_normal((1, 8, 16, D)).astype(np.float32)
    k = rng.standard_normal((1, 2, 16, D)).astype(np.float32)
    a = orc.gate_logits(q, k, w_in, b_in, w_out, bs)
    b = orc.gate_logits(q, np.repeat(k, 4, axis=1), w_in, b_in, w_out, bs)
    np.testing.assert_array_equal(a, b)


def test_threshold_mask_invariants():
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((2, 3, 6, 6)).astype(np.float32)
    soft, hard = orc.threshold_mask(logits, 0.5, causal=True)
    up = np.triu(np.ones((6, 6), bool), 1)
    assert (soft[..., up] == 0.0).all() and not hard[..., up].any()
    lo = ~up
    ref = torch.sigmoid(torch.from_numpy(logits)).numpy()
    np.testing.assert_allclose(soft[..., lo], ref[..., lo], rtol=1e-6)
    _, hard0 = orc.threshold_mask(logits, 0.0, causal=True)
    assert hard0.all()  # tau=0: 0 >= 0 in the upper triangle (test_edge_cases.py:210-218)
    _, hard1 = orc.threshold_mask(logits, 1.0 + 1e-7, causal=True)
    assert not hard1.any()
    soft_nc, _ = orc.threshold_mask(logits, 0.5, causal=False)
    assert (soft_nc[..., up] > 0).all()
    taus = np.array([0.2, 0.5, 0.9], dtype=np.float32)
    _, hh = orc.threshold_mask(logits, taus, causal=False)
    for h in range(3):
        np.testing.assert_array_equal(hh[:, h], soft_nc[:, h] >= taus[h])


# ----------------------------------------------------------------------------- attention
def _brute_attention(q, k, v, mask, bs, causal, scale):
    """Pure-Python loops: one query at a time, explicit max/exp/sum."""
    B, H, S, D = q.shape
    Sk = k.shape[2]
    g = H // k.shape[1]
    out = np.zeros_like(q, dtype=np.float64)
    for b in range(B):
        for h in range(H):
            for i in range(S):
                allowed = []
                for j in range(Sk):
                    if not mask[b, h, i // bs, j // bs]:
                        continue
                    if causal and (j // bs > i // bs or j > i):
                        continue
                    s = sum(float(q[b, h, i, d]) * float(k[b, h // g, j, d]) for d in range(D)) * scale
                    allowed.append((j, s))
                if not allowed:
                    continue
                m = max(s for _, s in allowed)
                w = [(j, math.exp(s - m)) for j, s in allowed]
                tot = sum(x for _, x in w)
                for d in range(D):
                    out[b, h, i, d] = sum(x * float(v[b, h // g, j, d]) for j, x in w) / tot
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_attention_matches_brute_force(causal):
    rng = np.random.default_rng(6)
    B, H, Hkv, S, D, bs = 1, 4, 2, 11, 3, 4
    q = rng.standard_normal((B, H, S, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    nb = math.ceil(S / bs)
    mask = rng.random((B, H, nb, nb)) < 0.6
    mask[0, 1, 1, :] = False  # an empty block row -> zeros
    ref = _brute_attention(q, k, v, mask, bs, causal, 0.7)
    for fn in (orc.attention_dense_masked, orc.attention_block_gather):
        got = fn(q, k, v, mask, bs, causal=causal, scale=0.7, dtype=np.float64)
        np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)
    assert (orc.attention_dense_masked(q, k, v, mask, bs, causal, 0.7)[0, 1, 4:8] == 0).all()


def _nan_pattern(q, k, v, mask, bs, causal):
    """Where the reference kernel's output is NaN (block_sparse_fa.py:215-257): a NaN score
    among a row's allowed keys makes p, l and the whole accumulator row NaN, and the division
    by ``where(l > 0, l, 1)`` keeps it (a NaN score at a masked element is replaced by -inf,
    :243). V is multiplied per active block (:252), so a NaN in V[j, d] reaches column d of
    every row whose block row has key j's block active, also where the element mask gives
    p = 0 (0 * NaN is NaN). Explicit loops over the allowed keys and active blocks."""
    B, H, S, D = q.shape
    g = H // k.shape[1]
    out = np.zeros(q.shape, dtype=bool)
    for b in range(B):
        for h in range(H):
            for i in range(S):
                in_block = [j for j in range(k.shape[2]) if mask[b, h, i // bs, j // bs]
                            and not (causal and j // bs > i // bs)]
                allowed = [j for j in in_block if not (causal and j > i)]
                if not allowed:
                    continue
                if np.isnan(q[b, h, i]).any() or any(np.isnan(k[b, h // g, j]).any() for j in allowed):
                    out[b, h, i] = True
                    continue
                for j in in_block:
                    out[b, h, i] |= np.isnan(v[b, h // g, j])
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_attention_nan_follows_reference_normalisation(causal):
    """NaN in Q, K or V propagates as in the reference kernel; empty rows stay exactly 0.
    The block-gather oracle (the checker of the kernels) follows the kernel's per-block V
    product; the dense oracle agrees when no inactive key of V holds a NaN."""
    rng = np.random.default_rng(16)
    B, H, Hkv, S, D, bs = 1, 4, 2, 13, 5, 4
    q = rng.standard_normal((B, H, S, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    q[0, 0, 6, 2] = np.nan
    k[0, 1, 3, 0] = np.nan
    v[0, 0, 9, 4] = np.nan
    nb = math.ceil(S / bs)
    mask = rng.random((B, H, nb, nb)) < 0.6
    mask[0, 3, 1, :] = False  # an empty block row
    want = _nan_pattern(q, k, v, mask, bs, causal)
    assert want.any() and not want.all()
    got = orc.attention_block_gather(q, k, v, mask, bs, causal=causal)
    np.testing.assert_array_equal(np.isnan(got), want)
    assert (got[0, 3, 4:8] == 0).all()
    clean = ~want
    ref = orc.attention_block_gather(np.nan_to_num(q), np.nan_to_num(k), np.nan_to_num(v), mask, bs,
                                     causal)
    # Rows and columns that no NaN reaches are unchanged by it.
    np.testing.assert_allclose(got[clean], ref[clean], rtol=1e-6, atol=1e-7)
    v2 = np.nan_to_num(v)
    want2 = _nan_pattern(q, k, v2, mask, bs, causal)
    dense = orc.attention_dense_masked(q, k, v2, mask, bs, causal=causal)
    np.testing.assert_array_equal(np.isnan(dense), want2)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_all_true_mask_equals_sdpa(causal):
    rng = np.random.default_rng(7)
    q = rng.standard_normal((2, 4, 70, 16)).astype(np.float32)
    k = rng.standard_normal((2, 4, 70, 16)).astype(np.float32)
    v = rng.standard_normal((2, 4, 70, 16)).astype(np.float32)
    mask = np.ones((2, 4, 3, 3), dtype=bool)
    got = orc.attention_block_gather(q, k, v, mask, 32, causal=causal, dtype=np.float64)
    ref = F.scaled_dot_product_attention(torch.from_numpy(q).double(), torch.from_numpy(k).double(),
                                         torch.from_numpy(v).double(), is_causal=causal).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_attention_gather_equals_dense_masked_gqa():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((1, 8, 200, 32)).astype(np.float32)
    k = rng.standard_normal((1, 2, 200, 32)).astype(np.float32)
    v = rng.standard_normal((1, 2, 200, 32)).astype(np.float32)
    mask = rng.random((1, 8, 4, 4)) < 0.5
    a = orc.attention_dense_masked(q, k, v, mask, 64, True, dtype=np.float64)
    b = orc.attention_block_gather(q, k, v, mask, 64, True, dtype=np.float64)
    np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_varlen_equals_block_diagonal_dense(causal):
    """Packed sequences == one dense masked attention over all tokens whose token mask is
    block-diagonal by sequence (built here element by element, not by the oracle)."""
    rng = np.random.default_rng(21)
    Hq, Hkv, D, bs = 4, 2, 16, 32
    cu = [0, 37, 37, 130, 200]  # an empty and a ragged sequence; tokens 200..207 unused
    T = 208
    nbmax = 4
    q = rng.standard_normal((T, Hq, D)).astype(np.float32)
    k = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    mask = rng.random((len(cu) - 1, Hq, nbmax, nbmax)) < 0.6
    got = orc.attention_varlen(q, k, v, cu, mask, bs, causal, dtype=np.float64)
    ref = np.zeros((T, Hq, D))
    sc = 1 / math.sqrt(D)
    for h in range(Hq):
        allow = np.zeros((T, T), dtype=bool)
        for n in range(len(cu) - 1):
            for i in range(cu[n], cu[n + 1]):
                for j in range(cu[n], cu[n + 1]):
                    bi, bj = (i - cu[n]) // bs, (j - cu[n]) // bs
                    allow[i, j] = mask[n, h, bi, bj] and (not causal or j <= i)
        sco = (q[:, h].astype(np.float64) @ k[:, h // 2].astype(np.float64).T) * sc
        for i in range(T):
            if allow[i].any():
                row = np.where(allow[i], sco[i], -np.inf)
                p_ = np.exp(row - row.max())
                ref[i, h] = (p_ / p_.sum()) @ v[:, h // 2].astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)
    assert (got[200:] == 0).all()


def test_attention_varlen_single_sequence_is_flat_token_call():
    """One packed sequence is the reference's flat-token view (B = 1, vllm_patch.py:172-176)."""
    rng = np.random.default_rng(22)
    T, Hq, Hkv, D, bs = 150, 4, 1, 8, 64
    q = rng.standard_normal((T, Hq, D)).astype(np.float32)
    k = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    mask = rng.random((1, Hq, 3, 3)) < 0.7
    got = orc.attention_varlen(q, k, v, [0, T], mask, bs, True, dtype=np.float64)
    flat = orc.attention_dense_masked(q.transpose(1, 0, 2)[None], k.transpose(1, 0, 2)[None],
                                      v.transpose(1, 0, 2)[None], mask, bs, True, dtype=np.float64)
    np.testing.assert_allclose(got, flat[0].transpose(1, 0, 2), rtol=1e-10, atol=1e-12)


# ----------------------------------------------------------------------------- decode
def test_decode_equals_last_prefill_row_and_brute_force():
    rng = np.random.default_rng(9)
    B, H, Hkv, S, D, bs = 2, 4, 2, 100, 8, 16
    q_all = rng.standard_normal((B, H, S, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    nb = math.ceil(S / bs)
    row = rng.random((B, H, 1, nb)) < 0.5
    row[0, 0, 0, :] = False  # head with nothing selected -> 0
    full = np.zeros((B, H, nb, nb), dtype=bool)
    full[:, :, nb - 1, :] = row[:, :, 0, :]
    pre = orc.attention_block_gather(q_all, k, v, full, bs, causal=True, dtype=np.float64)
    dec = orc.sparse_decode(q_all[:, :, S - 1 : S], k, v, row, bs, dtype=np.float64)
    np.testing.assert_allclose(dec[:, :, 0], pre[:, :, S - 1], rtol=1e-10, atol=1e-12)
    assert (dec[0, 0] == 0).all()
    brute = _brute_attention(q_all[:, :, S - 1 : S], k[:, :, :S], v, np.repeat(row, 1, axis=2), bs,
                             False, 1 / math.sqrt(D))
    np.testing.assert_allclose(dec, brute, rtol=1e-10, atol=1e-12)


def test_decode_paged_equals_contiguous_cache():
    """Pools scattered from a contiguous cache through a random page permutation."""
    rng = np.random.default_rng(23)
    B, H, Hkv, S, D, bs, ps = 3, 4, 2, 128, 8, 32, 16
    q = rng.standard_normal((B, H, 1, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    lens = np.array([128, 77, 16])
    mask = rng.random((B, H, 1, S // bs)) < 0.6
    per = S // ps
    perm = rng.permutation(B * per + 5)  # spare pages stay unused
    table = perm[: B * per].reshape(B, per)
    kp = rng.standard_normal((B * per + 5, ps, Hkv, D)).astype(np.float32)
    vp = rng.standard_normal((B * per + 5, ps, Hkv, D)).astype(np.float32)
    for b in range(B):
        for j in range(per):
            kp[table[b, j]] = k[b, :, j * ps:(j + 1) * ps].transpose(1, 0, 2)
            vp[table[b, j]] = v[b, :, j * ps:(j + 1) * ps].transpose(1, 0, 2)
    got = orc.sparse_decode_paged(q, kp, vp, table, lens, mask, bs, dtype=np.float64)
    ref = orc.sparse_decode(q, k, v, mask, bs, lens, dtype=np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-14)


def test_decode_kv_lens_equals_truncated_cache():
    rng = np.random.default_rng(10)
    q = rng.standard_normal((2, 2, 1, 8)).astype(np.float32)
    k = rng.standard_normal((2, 1, 64, 8)).astype(np.float32)
    v = rng.standard_normal((2, 1, 64, 8)).astype(np.float32)
    m = np.ones((2, 2, 1, 4), dtype=bool)
    got = orc.sparse_decode(q, k, v, m, 16, kv_lens=[37, 64], dtype=np.float64)
    ref0 = orc.sparse_decode(q[:1], k[:1, :, :37], v[:1, :, :37], m[:1, :, :, :3], 16, dtype=np.float64)
    np.testing.assert_allclose(got[:1], ref0, rtol=1e-12)


# ----------------------------------------------------------------------------- gate target from q, k
@pytest.mark.parametrize("causal", [True, False])
def test_block_max_equals_explicit_scores(causal):
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 4, 45, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 45, 8)).astype(np.float32)
    sc = 0.3
    kk = np.repeat(k, 2, axis=1)
    scores = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), kk.astype(np.float64)) * sc
    if causal:
        scores = scores + np.triu(np.full((45, 45), -np.inf), 1)
    ref = orc.gate_target_from_scores(scores, 16)
    got = orc.gate_target_from_qk(q, k, 16, causal=causal, scale=sc)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-9)
    row = orc.gate_target_from_qk(q, k, 16, causal=causal, scale=sc, normalize="row")
    np.testing.assert_allclose(row.sum(-1), 1.0, rtol=1e-12)


@pytest.mark.parametrize("form", ["padding_2d", "binary_2d", "hf_4d", "per_head_4d"])
def test_block_max_with_attention_mask_equals_reference_composition(form):
    """Scores built as tasft_attention.py:426-449 does (torch: matmul * scale, + triu(-inf),
    + attention_mask with a 2-D mask broadcast as [:, None, None, :]), then the reference
    pooling path, against the oracle's fused block maxima."""
    rng = np.random.default_rng(12)
    B, H, Hkv, S, D, bs = 2, 4, 2, 45, 8, 16
    q = rng.standard_normal((B, H, S, D)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
    sc = 0.3
    lens = [45, 30]
    if form == "padding_2d":
        mask = np.zeros((B, S), dtype=np.float32)
        mask[1, 30:] = -np.inf
    elif form == "binary_2d":
        mask = (np.arange(S)[None, :] < np.array(lens)[:, None]).astype(np.float32)  # 1 keep, 0 pad
    elif form == "hf_4d":
        fmin = np.finfo(np.float32).min
        allowed = (np.arange(S)[None, None, :] <= np.arange(S)[None, :, None]) & \
                  (np.arange(S)[None, None, :] < np.array(lens)[:, None, None])
        mask = np.where(allowed, 0.0, fmin).astype(np.float32)[:, None]  # [B, 1, S, S]
    else:
        mask = rng.standard_normal((B, H, S, S)).astype(np.float32)
    qt, kt = torch.from_numpy(q).double(), torch.from_numpy(k).double().repeat_interleave(2, dim=1)
    weights = torch.matmul(qt, kt.transpose(-2, -1)) * sc
    weights = weights + torch.triu(torch.full((S, S), float("-inf"), dtype=torch.float64), 1)[None, None]
    ext = torch.from_numpy(mask).double()
    if ext.ndim == 2:
        ext = ext[:, None, None, :]
    weights = weights + ext
    ref = orc.gate_target_from_scores(weights.numpy(), bs)
    got = orc.gate_target_from_qk(q, k, bs, causal=True, scale=sc, attn_mask=mask)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-9)
    raw = orc.block_max(q, k, bs, True, sc, attn_mask=mask)
    nb = raw.shape[-1]
    pooled = torch.nn.functional.max_pool2d(
        torch.nn.functional.pad(weights, (0, nb * bs - S, 0, nb * bs - S), value=-math.inf), bs, bs)
    np.testing.assert_allclose(raw, pooled.numpy(), rtol=1e-5, atol=1e-6)


def _kl_case(seed):
    rng = np.random.default_rng(seed)
    soft = 1.0 / (1.0 + np.exp(-rng.standard_normal((2, 3, 5, 5))))
    soft = soft * np.tril(np.ones((5, 5)))  # causal zeros, as the gate produces
    target = orc.gate_target_from_scores(rng.standard_normal((2, 3, 20, 20)) * 3, 4)
    target[0, 0, 1, :] = 0.0  # exact zeros in the target
    target[0, 0] /= target[0, 0].sum()
    return soft, target


def test_gate_kl_loss_matches_reference_kl_div_composition():
    """objectives.py:210-221 composed with torch: normalise, log(. + eps), F.kl_div batchmean."""
    soft, target = _kl_case(21)
    st = torch.from_numpy(soft)
    tt = torch.from_numpy(target)
    b, h = st.shape[:2]
    flat = st.reshape(b, h, -1)
    dist = flat / (flat.sum(-1, keepdim=True) + 1e-8)
    ref = torch.nn.functional.kl_div(torch.log(dist + 1e-8), tt.reshape(b, h, -1),
                                     reduction="batchmean", log_target=False)
    assert orc.gate_kl_loss(soft, target) == pytest.approx(float(ref), rel=1e-12, abs=1e-14)


def test_gate_kl_grad_matches_autograd():
    soft, target = _kl_case(22)
    st = torch.from_numpy(soft).requires_grad_(True)
    b, h = st.shape[:2]
    flat = st.reshape(b, h, -1)
    dist = flat / (flat.sum(-1, keepdim=True) + 1e-8)
    loss = torch.nn.functional.kl_div(torch.log(dist + 1e-8), torch.from_numpy(target).reshape(b, h, -1),
                                      reduction="batchmean", log_target=False)
    loss.backward()
    np.testing.assert_allclose(orc.gate_kl_grad(soft, target), st.grad.numpy(), rtol=1e-9, atol=1e-12)


def test_gate_target_clamp_temperature_variant():
    pooled = np.array([[[[100.0, -np.inf], [3.0, -70.0]]]])
    got = orc.normalize_block_max(pooled, "flat", temperature=2.0, clamp=50.0)
    ref = torch.softmax(torch.tensor([50.0, -math.inf, 3.0, -50.0], dtype=torch.float64) / 2.0, 0)
    np.testing.assert_allclose(got.reshape(-1), ref.numpy(), rtol=1e-12)


def test_mask_csr_literal_and_round_trip():
    # Hand-checked: rows (b=0,h=0,qb=0..2) of a 3x4 mask.
    mask = np.array([[[[1, 0, 1, 0], [0, 0, 0, 0], [1, 1, 0, 1]]]], dtype=np.uint8)
    rp, ci = orc.mask_to_csr(mask)
    assert rp.tolist() == [0, 2, 2, 5]
    assert ci.tolist() == [0, 2, 0, 1, 3]
    rp_c, ci_c = orc.mask_to_csr(mask, causal=True)  # keeps kb <= qb
    assert rp_c.tolist() == [0, 1, 1, 3]
    assert ci_c.tolist() == [0, 0, 1]
    rng = np.random.default_rng(5)
    m = rng.random((2, 3, 7, 9)) < 0.3
    rp, ci = orc.mask_to_csr(m)
    back = np.zeros((2 * 3 * 7, 9), dtype=bool)
    for r in range(back.shape[0]):
        back[r, ci[rp[r]:rp[r + 1]]] = True
    assert np.array_equal(back.reshape(m.shape), m)


def test_indices_to_mask_literal():
    idx = np.array([[[3, -1, 0, 3]], [[-1, -1, -1, -1]]], dtype=np.int32)  # [2, 1, 4]
    m = orc.indices_to_mask(idx, 5)
    assert m.shape == (2, 1, 5)
    assert m[0, 0].tolist() == [True, False, False, True, False]
    assert not m[1].any()
