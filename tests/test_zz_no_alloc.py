"""tasft_bsfa_decode_fwd_noalloc: the decode variant that allocates nothing.

It keeps the split partials in the library's static device scratch instead of a caller
workspace. Called through the C ABI, its output must equal tasft_bsfa_decode_fwd's bit for
bit (same kernels) on two calls in a row, the second one smaller, and meet the parity bar
against the oracle; sizes beyond the scratch are rejected before any launch.
"""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

import attn_inputs as ai
from helpers import assert_close_bf16, require_gpu, to_np
from oracle import tasft_oracle as orc
from tasft_amd import _native

pytestmark = pytest.mark.gpu


def _args(q, kc, vc, out, mask, lens, splits, bs):
    B, Hq, _, D = q.shape
    return (q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), mask.data_ptr(),
            _native.ptr(lens)), (B, Hq, kc.shape[1], kc.shape[2], D, bs, splits,
                                 _native.strides(q), _native.strides(kc), _native.strides(vc),
                                 _native.strides(out), _native.strides(mask),
                                 ctypes.c_float(1.0 / math.sqrt(D)),
                                 _native.dtype_code(q.dtype, "decode"), _native.stream_handle(q.device))


def _decode_both(case, kind, dev):
    B, Hq, Hkv, S, D, bs, _dens, splits = case
    q, kc, vc, mask = ai.decode_case_inputs(case, kind)
    lens = torch.randint(1, S + 1, (B,), generator=torch.Generator().manual_seed(S)).to(torch.int32)
    qd, kd, vd, md, ld = q.to(dev), kc.to(dev), vc.to(dev), mask.view(torch.uint8).to(dev), lens.to(dev)
    lib = _native.load_library()
    need = lib.tasft_bsfa_decode_workspace_bytes(B, Hq, D, splits)
    assert 0 < need <= _native.DECODE_NOALLOC_MAX_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    ref_out = torch.empty_like(qd)
    ptrs, rest = _args(qd, kd, vd, ref_out, md, ld, splits, bs)
    rc = lib.tasft_bsfa_decode_fwd(*ptrs, ws.data_ptr(), need, *rest)
    _native.check(rc, "tasft_bsfa_decode_fwd")
    out = torch.empty_like(qd)
    ptrs, rest = _args(qd, kd, vd, out, md, ld, splits, bs)
    rc = lib.tasft_bsfa_decode_fwd_noalloc(*ptrs, *rest)
    _native.check(rc, "tasft_bsfa_decode_fwd_noalloc")
    torch.cuda.synchronize()
    ref = orc.sparse_decode(to_np(q), to_np(kc), to_np(vc), mask.numpy(), bs, kv_lens=lens.numpy())
    return out, ref_out, ref


def test_noalloc_decode_equals_workspace_decode_twice_second_smaller():
    dev = require_gpu()
    big = (4, 32, 8, 4096, 128, 64, 0.2, 8)     # 532 KB of partials
    small = (2, 8, 2, 1000, 64, 32, 0.4, 3)     # a later, smaller call on the same scratch
    for case in (big, small):
        print(f"noalloc decode {case}", flush=True)
        out, ref_out, ref = _decode_both(case, "unit", dev)
        assert torch.equal(out, ref_out), f"{case}: no-alloc output differs from the workspace call"
        assert_close_bf16(out, ref, f"noalloc decode {case}")


def test_noalloc_decode_rejects_partials_beyond_the_scratch():
    dev = require_gpu()
    lib = _native.load_library()
    B, Hq, Hkv, S, D, bs, splits = 64, 32, 8, 32768, 128, 64, 64
    need = lib.tasft_bsfa_decode_workspace_bytes(B, Hq, D, splits)
    assert need > _native.DECODE_NOALLOC_MAX_BYTES
    q = torch.zeros(B, Hq, 1, D, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(1, 1, 1, D, dtype=torch.bfloat16, device=dev).expand(B, Hkv, S, D)
    mask = torch.zeros(B, Hq, 1, S // bs, dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)
    ptrs, rest = _args(q, kc, kc, out, mask, None, splits, bs)
    rc = lib.tasft_bsfa_decode_fwd_noalloc(*ptrs, *rest)
    assert rc == -4
    assert b"static scratch" in lib.tasft_last_error()
