"""The attention parity cases can tell a correct kernel from a broken one (CPU only).

For every case the GPU parity tests run on ``unit`` and ``peaky`` inputs
(``tests/attn_inputs.py``), three stand-ins for a kernel are compared with the oracle under
the same bar the GPU tests apply (``helpers.parity_failure``):

* uniform weights (the oracle with scale 0, i.e. a kernel whose softmax ignores QK^T),
  twice the scale (a wrong exp2 factor) and, for the prefill, query rows swapped in
  pairs inside every block before QK^T (a wrong score-fragment row mapping) must FAIL
  the bar;
* a bf16 emulation of the kernel arithmetic (P rounded to bf16 before PV, output rounded
  to bf16) must PASS it, so the bar is reachable.

The fp16 cases repeat this with fp16 inputs, the fp16 emulation and the tighter fp16 bar.

A further check shows that the benchmark-scale inputs (``base``) alone could not make
that distinction, which is why both kinds are tested.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import attn_inputs as ai
from helpers import bar, parity_failure, round_bf16, round_f16, to_np
from oracle import tasft_oracle as orc

DISC_KINDS = ("unit", "peaky")


def _emul_rows(qrows, keys, vals, allowed, scale, rnd=round_bf16):
    """Emulation of one head: rows of q against ``keys`` under ``allowed``, P and the
    output rounded by ``rnd`` (bf16 or fp16)."""
    sco = (qrows @ keys.T) * np.float32(scale)
    sco = np.where(allowed, sco, -np.inf)
    mx = sco.max(axis=-1, keepdims=True)
    has = np.isfinite(mx)
    p = np.exp(sco - np.where(has, mx, 0.0)).astype(np.float32)
    l = p.sum(axis=-1, keepdims=True)
    o = rnd(p) @ vals
    return rnd(np.where(l > 0, o / np.where(l > 0, l, 1.0), 0.0).astype(np.float32))


def _emul_prefill(q, k, v, mask, bs, causal, rnd=round_bf16):
    b_, hq, s, d = q.shape
    g = hq // k.shape[1]
    out = np.zeros(q.shape, dtype=np.float32)
    for b in range(b_):
        for h in range(hq):
            tm = orc.token_mask(mask[b, h], s, bs, causal)
            out[b, h] = _emul_rows(q[b, h], k[b, h // g], v[b, h // g], tm, 1.0 / math.sqrt(d), rnd)
    return out


def _emul_decode(q, kc, vc, mask, bs, kv_lens=None, rnd=round_bf16):
    b_, hq, _, d = q.shape
    g = hq // kc.shape[1]
    s = kc.shape[2]
    out = np.zeros(q.shape, dtype=np.float32)
    for b in range(b_):
        n = s if kv_lens is None else int(kv_lens[b])
        for h in range(hq):
            tok = np.repeat(mask[b, h, 0].astype(bool), bs)[:s] & (np.arange(s) < n)
            out[b, h, 0] = _emul_rows(q[b, h, :1], kc[b, h // g], vc[b, h // g], tok[None, :],
                                      1.0 / math.sqrt(d), rnd)[0]
    return out


def _swap_row_pairs(q):
    """Query rows 2i and 2i+1 exchanged along the token axis (axis -2)."""
    s = q.shape[-2]
    idx = np.arange(s)
    even = idx[: s - s % 2]
    idx[: s - s % 2] = even ^ 1
    return q[..., idx, :]


def _check(what, ref, uniform, double, emul, swapped=None, dtype=torch.bfloat16):
    kw = bar(dtype)
    assert parity_failure(uniform, ref, **kw) is not None, f"{what}: uniform weights pass the bar"
    assert parity_failure(double, ref, **kw) is not None, f"{what}: twice the scale passes the bar"
    if swapped is not None:
        assert parity_failure(swapped, ref, **kw) is not None, f"{what}: swapped query rows pass the bar"
    fail = parity_failure(emul, ref, **kw)
    assert fail is None, f"{what}: {dtype} emulation fails the bar: {fail}"


@pytest.mark.parametrize("kind", DISC_KINDS)
@pytest.mark.parametrize("case", ai.PREFILL_CASES, ids=ai.case_id)
def test_prefill_cases_discriminate(case, kind):
    _B, _Hq, _Hkv, _S, D, bs, causal, _dens, _var = case
    qt, kt, vt, mask = ai.prefill_case_inputs(case, kind)
    q, k, v, m = to_np(qt), to_np(kt), to_np(vt), mask.numpy()
    sc = 1.0 / math.sqrt(D)
    ref = orc.attention_block_gather(q, k, v, m, bs, causal)
    _check(f"prefill {case} {kind}", ref,
           orc.attention_block_gather(q, k, v, m, bs, causal, scale=0.0),
           orc.attention_block_gather(q, k, v, m, bs, causal, scale=2 * sc),
           _emul_prefill(q, k, v, m, bs, causal),
           orc.attention_block_gather(_swap_row_pairs(q), k, v, m, bs, causal))


@pytest.mark.parametrize("kind", DISC_KINDS)
@pytest.mark.parametrize("case", ai.VARLEN_CASES, ids=ai.case_id)
def test_varlen_cases_discriminate(case, kind):
    lens, _Hq, _Hkv, D, bs, causal, _dens = case
    q, k, v, cu, mask = ai.varlen_case_inputs(case, kind)
    qn, kn, vn, m = to_np(q), to_np(k), to_np(v), mask.numpy()
    sc = 1.0 / math.sqrt(D)
    ref = orc.attention_varlen(qn, kn, vn, cu, m, bs, causal)
    emul = np.zeros_like(ref)
    for n in range(len(lens)):
        t0, t1 = cu[n], cu[n + 1]
        if t1 > t0:
            nb = math.ceil((t1 - t0) / bs)
            o = _emul_prefill(qn[t0:t1].transpose(1, 0, 2)[None], kn[t0:t1].transpose(1, 0, 2)[None],
                              vn[t0:t1].transpose(1, 0, 2)[None], m[n:n + 1, :, :nb, :nb], bs, causal)
            emul[t0:t1] = o[0].transpose(1, 0, 2)
    _check(f"varlen {case} {kind}", ref,
           orc.attention_varlen(qn, kn, vn, cu, m, bs, causal, scale=0.0),
           orc.attention_varlen(qn, kn, vn, cu, m, bs, causal, scale=2 * sc), emul)


@pytest.mark.parametrize("kind", DISC_KINDS)
@pytest.mark.parametrize("case", ai.DECODE_CASES, ids=ai.case_id)
def test_decode_cases_discriminate(case, kind):
    D, bs = case[4], case[5]
    q, kc, vc, mask = ai.decode_case_inputs(case, kind)
    qn, kn, vn, m = to_np(q), to_np(kc), to_np(vc), mask.numpy()
    sc = 1.0 / math.sqrt(D)
    ref = orc.sparse_decode(qn, kn, vn, m, bs)
    _check(f"decode {case} {kind}", ref,
           orc.sparse_decode(qn, kn, vn, m, bs, scale=0.0),
           orc.sparse_decode(qn, kn, vn, m, bs, scale=2 * sc),
           _emul_decode(qn, kn, vn, m, bs))


@pytest.mark.parametrize("kind", DISC_KINDS)
@pytest.mark.parametrize("case", ai.PAGED_CASES, ids=ai.case_id)
def test_paged_cases_discriminate(case, kind):
    D, bs = case[4], case[5]
    q, k, v, kp, vp, table, lens, mask = ai.paged_case_inputs(case, kind)
    qn, m, ln = to_np(q), mask.numpy(), lens.numpy()
    kpn, vpn, tn = to_np(kp), to_np(vp), table.numpy()
    sc = 1.0 / math.sqrt(D)
    ref = orc.sparse_decode_paged(qn, kpn, vpn, tn, ln, m, bs)
    _check(f"paged {case} {kind}", ref,
           orc.sparse_decode_paged(qn, kpn, vpn, tn, ln, m, bs, scale=0.0),
           orc.sparse_decode_paged(qn, kpn, vpn, tn, ln, m, bs, scale=2 * sc),
           _emul_decode(qn, to_np(k), to_np(v), m, bs, kv_lens=ln))


@pytest.mark.parametrize("kind", DISC_KINDS)
@pytest.mark.parametrize("case", ai.F16_PREFILL_CASES, ids=ai.case_id)
def test_f16_prefill_cases_discriminate(case, kind):
    """fp16 inputs: the fp16 emulation meets the fp16 bar, the broken stand-ins do not."""
    _B, _Hq, _Hkv, _S, D, bs, causal, _dens, _var = case
    qt, kt, vt, mask = ai.prefill_case_inputs(case, kind, torch.float16)
    q, k, v, m = to_np(qt), to_np(kt), to_np(vt), mask.numpy()
    sc = 1.0 / math.sqrt(D)
    ref = orc.attention_block_gather(q, k, v, m, bs, causal)
    _check(f"fp16 prefill {case} {kind}", ref,
           orc.attention_block_gather(q, k, v, m, bs, causal, scale=0.0),
           orc.attention_block_gather(q, k, v, m, bs, causal, scale=2 * sc),
           _emul_prefill(q, k, v, m, bs, causal, round_f16),
           orc.attention_block_gather(_swap_row_pairs(q), k, v, m, bs, causal), torch.float16)


@pytest.mark.parametrize("kind", DISC_KINDS)
@pytest.mark.parametrize("case", ai.F16_DECODE_CASES, ids=ai.case_id)
def test_f16_decode_cases_discriminate(case, kind):
    D, bs = case[4], case[5]
    q, kc, vc, mask = ai.decode_case_inputs(case, kind, torch.float16)
    qn, kn, vn, m = to_np(q), to_np(kc), to_np(vc), mask.numpy()
    sc = 1.0 / math.sqrt(D)
    ref = orc.sparse_decode(qn, kn, vn, m, bs)
    _check(f"fp16 decode {case} {kind}", ref,
           orc.sparse_decode(qn, kn, vn, m, bs, scale=0.0),
           orc.sparse_decode(qn, kn, vn, m, bs, scale=2 * sc),
           _emul_decode(qn, kn, vn, m, bs, rnd=round_f16), dtype=torch.float16)


def test_peaky_inputs_move_the_running_maximum():
    """In every peaky prefill row that spans several key blocks, some later block's scores
    exceed the maximum of all earlier blocks by more than 8 log2 units."""
    case = ai.PREFILL_CASES[0]
    q, k, _v, _mask = ai.prefill_case_inputs(case, "peaky")
    qn, kn = to_np(q)[0, 0], to_np(k)[0, 0]
    bs = case[5]
    s = (qn @ kn.T) / math.sqrt(case[4]) * math.log2(math.e)
    rows = np.arange(4 * bs, s.shape[0], 97)
    for r in rows:
        nblk = r // bs + 1
        blk_max = [s[r, j * bs:min((j + 1) * bs, r + 1)].max() for j in range(nblk)]
        jumps = [blk_max[j] - max(blk_max[:j]) for j in range(1, nblk)]
        assert max(jumps) > 8.0, f"row {r}: largest jump {max(jumps):.2f} log2 units"


def test_base_scale_inputs_alone_do_not_discriminate():
    """At N(0,1)/sqrt(128) a uniform-weight kernel meets the absolute bar: the reason the
    parity tests add the unit and peaky kinds."""
    case = ai.PREFILL_CASES[0]
    q, k, v, mask = ai.prefill_case_inputs(case, "base")
    qn, kn, vn, m = to_np(q), to_np(k), to_np(v), mask.numpy()
    ref = orc.attention_block_gather(qn, kn, vn, m, case[5], True)
    uni = orc.attention_block_gather(qn, kn, vn, m, case[5], True, scale=0.0)
    assert parity_failure(uni, ref, rel=None) is None
