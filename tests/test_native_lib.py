"""The C-ABI library loads on the CPU and exports every symbol the header declares.

Only host-side entry points are called here (version, workspace sizes, argument
validation that returns before any device work); no kernel is launched.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from tasft_amd import _native

HEADER = Path(__file__).resolve().parent.parent / "include" / "tasft_amd.h"


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(tasft_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _native.load_library()
    declared = _declared_functions()
    assert declared, "no declarations parsed from the header"
    assert declared == set(_native.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), f"{name} missing from {_native.LIB_PATH}"


def test_abi_version_and_workspace_sizes():
    lib = _native.load_library()
    assert lib.tasft_abi_version() == 9
    assert lib.tasft_bsfa_prefill_workspace_bytes(4, 32, 8192, 64) == 256
    assert lib.tasft_bsfa_prefill_workspace_bytes(4, 32, 0, 64) == 0
    assert lib.tasft_bsfa_decode_workspace_bytes(64, 32, 128, 4) == 64 * 32 * 4 * 130 * 4
    assert lib.tasft_bsfa_decode_workspace_bytes(0, 32, 128, 4) == 0
    nb = 8192 // 64
    # Projected units, then one 64-byte completion counter per (b, KV head).
    assert lib.tasft_gate_workspace_bytes(4, 32, 8, 8192, 128, 64, 128) == 4 * 40 * nb * 128 * 4 + 4 * 8 * 64
    assert lib.tasft_gate_workspace_bytes(4, 32, 8, 8192, 0, 64, 128) == 0
    assert lib.tasft_mask_compact_workspace_bytes(4, 32, 128) == 4 * 32 * 128 * 4
    assert lib.tasft_mask_compact_workspace_bytes(0, 32, 128) == 0


def _i64(vals):
    return (ctypes.c_int64 * 4)(*vals)


def test_invalid_arguments_return_errors_without_launch():
    lib = _native.load_library()
    st = _i64([0, 0, 0, 1])
    rc = lib.tasft_bsfa_prefill_fwd(None, None, None, None, None, None, 0, 1, 32, 8, 128, 128, 64,
                                    st, st, st, st, st, 1.0, 1, 0, None)
    assert rc == -1 and b"null pointer" in lib.tasft_last_error()
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.tasft_bsfa_prefill_fwd(fake, fake, fake, fake, fake, None, 0, 1, 32, 8, 128, 96, 64,
                                    st, st, st, st, st, 1.0, 1, 0, None)
    assert rc == -2 and b"head_dim" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_prefill_fwd(fake, fake, fake, fake, fake, None, 0, 1, 30, 8, 128, 128, 64,
                                    st, st, st, st, st, 1.0, 1, 0, None)
    assert rc == -1 and b"multiple" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_prefill_fwd(fake, fake, fake, fake, fake, fake, 16, 1, 32, 8, 128, 128, 64,
                                    st, st, st, st, st, 1.0, 1, 0, None)
    assert rc == -4 and b"workspace" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_decode_fwd(fake, fake, fake, fake, fake, None, fake, 0, 1, 32, 8, 1024, 128,
                                   64, 4, st, st, st, st, st, 1.0, 0, None)
    assert rc == -4 and b"workspace" in lib.tasft_last_error()
    rc = lib.tasft_mask_compact(fake, 1, 1, 4, 4, st, 0, fake, fake, 16, fake, 0, None)
    assert rc == -4 and b"workspace" in lib.tasft_last_error()
    rc = lib.tasft_mask_from_indices(fake, 4, 3, 2, 10, fake, fake, None)
    assert rc == -1 and b"invalid sizes" in lib.tasft_last_error()
    st3 = _i64([0, 0, 1])
    rc = lib.tasft_bsfa_prefill_varlen_fwd(fake, fake, fake, fake, fake, None, 2, 32, 8, 128, 128,
                                           64, st3, st3, st3, st3, st, 1.0, 1, 0, None)
    assert rc == -1 and b"null pointer" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_prefill_varlen_fwd(fake, fake, fake, fake, fake, fake, 2, 32, 8, 128, 128,
                                           48, st3, st3, st3, st3, st, 1.0, 1, 0, None)
    assert rc == -2 and b"block_size" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_prefill_varlen_fwd(fake, fake, fake, fake, fake, fake, 2, 32, 8, 128, 128,
                                           64, _i64([8, 8, 2]), st3, st3, st3, st, 1.0, 1, 0, None)
    assert rc == -1 and b"contiguous" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_varlen_zero_tail(None, fake, 2, 100, 32, 128, _i64([4096, 128, 1]), None)
    assert rc == -1 and b"null pointer" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_varlen_zero_tail(fake, fake, 2, 100, 32, 12, _i64([384, 12, 1]), None)
    assert rc == -1 and b"multiple of 8" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_varlen_zero_tail(fake, fake, 2, 100, 32, 128, _i64([4096, 128, 2]), None)
    assert rc == -1 and b"contiguous" in lib.tasft_last_error()
    assert lib.tasft_bsfa_varlen_zero_tail(fake, fake, 2, 0, 32, 128, _i64([4096, 128, 1]), None) == 0
    rc = lib.tasft_bsfa_decode_paged_fwd(fake, fake, fake, fake, fake, fake, fake, fake, 0, 1, 32,
                                         8, 1024, 128, 256, 16, 100, 4, st, st, st, st, st, 64, 1.0, 0, None)
    assert rc == -2 and b"block_size" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_decode_paged_fwd(fake, fake, fake, fake, fake, fake, fake, fake, 0, 1, 32,
                                         8, 1024, 128, 64, 12, 100, 4, st, st, st, st, st, 64, 1.0, 0, None)
    assert rc == -2 and b"page_size" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_decode_paged_fwd(fake, fake, fake, fake, fake, fake, fake, fake, 0, 1, 32,
                                         8, 1024, 128, 64, 16, 100, 4, st, st, st, st, st, 64, 1.0, 0, None)
    assert rc == -4 and b"workspace" in lib.tasft_last_error()
    rc = lib.tasft_bsfa_decode_paged_fwd(fake, fake, fake, fake, fake, fake, fake, fake, 1 << 20, 1, 32,
                                         8, 1024, 128, 64, 16, 0, 4, st, st, st, st, st, 64, 1.0, 0, None)
    assert rc == -1 and b"positive" in lib.tasft_last_error()


def test_dtype_codes_other_than_bf16_and_fp16_are_rejected():
    lib = _native.load_library()
    st = _i64([0, 0, 0, 1])
    st3 = _i64([0, 0, 1])
    fake = ctypes.c_void_p(16)
    calls = {
        "prefill": lambda dt: lib.tasft_bsfa_prefill_fwd(
            fake, fake, fake, fake, fake, None, 0, 1, 32, 8, 128, 128, 64, st, st, st, st, st, 1.0, 1,
            dt, None),
        "prefill_varlen": lambda dt: lib.tasft_bsfa_prefill_varlen_fwd(
            fake, fake, fake, fake, fake, fake, 2, 32, 8, 128, 128, 64, st3, st3, st3, st3, st, 1.0,
            1, dt, None),
        "decode": lambda dt: lib.tasft_bsfa_decode_fwd(
            fake, fake, fake, fake, fake, None, fake, 1 << 20, 1, 32, 8, 1024, 128, 64, 4, st, st, st,
            st, st, 1.0, dt, None),
        "decode_noalloc": lambda dt: lib.tasft_bsfa_decode_fwd_noalloc(
            fake, fake, fake, fake, fake, None, 1, 32, 8, 1024, 128, 64, 4, st, st, st, st, st, 1.0,
            dt, None),
        "decode_paged": lambda dt: lib.tasft_bsfa_decode_paged_fwd(
            fake, fake, fake, fake, fake, fake, fake, fake, 1 << 20, 1, 32, 8, 1024, 128, 64, 16, 100,
            4, st, st, st, st, st, 64, 1.0, dt, None),
        "gate": lambda dt: lib.tasft_gate_fwd(
            fake, fake, fake, fake, fake, fake, fake, None, fake, fake, None, None, fake, 1 << 20, 1,
            32, 8, 1024, 128, 64, 128, st, st, 1, dt, None),
        "gate_target": lambda dt: lib.tasft_gate_target_fwd(
            fake, fake, None, fake, 1, 32, 8, 1024, 128, 64, st, st, None, 1.0, 1, 0, 1.0, 0.0, dt,
            None),
        "gate_decode_rows": lambda dt: lib.tasft_gate_decode_rows_fwd(
            fake, fake, st, st, fake, fake, fake, 4096, fake, fake, fake, fake, fake, fake, fake,
            fake, 1, 32, 8, 128, 128, 3, 0, 2, dt, None),
    }
    for name, call in calls.items():
        for dt in (2, -1):
            rc = call(dt)
            assert rc == -2 and b"dtype" in lib.tasft_last_error(), name


def test_negative_strides_are_rejected_before_any_launch():
    """Every strided entry point refuses a negative stride (the kernels index forward from
    each tensor's base pointer) with an argument error, without touching the GPU."""
    lib = _native.load_library()
    st, neg = _i64([0, 0, 0, 1]), _i64([-8, 0, 0, 1])
    st3, neg3 = _i64([0, 0, 1]), _i64([-8, 0, 1])
    fake = ctypes.c_void_p(16)
    calls = {
        "prefill": lambda s4, s3, m: lib.tasft_bsfa_prefill_fwd(
            fake, fake, fake, fake, fake, None, 0, 1, 32, 8, 128, 128, 64, s4, st, st, st, m, 1.0,
            1, 0, None),
        "prefill_varlen": lambda s4, s3, m: lib.tasft_bsfa_prefill_varlen_fwd(
            fake, fake, fake, fake, fake, fake, 2, 32, 8, 128, 128, 64, st3, s3, st3, st3, m, 1.0,
            1, 0, None),
        "decode": lambda s4, s3, m: lib.tasft_bsfa_decode_fwd(
            fake, fake, fake, fake, fake, None, fake, 1 << 20, 1, 32, 8, 1024, 128, 64, 4, st, s4,
            st, st, m, 1.0, 0, None),
        "decode_paged": lambda s4, s3, m: lib.tasft_bsfa_decode_paged_fwd(
            fake, fake, fake, fake, fake, fake, fake, fake, 1 << 20, 1, 32, 8, 1024, 128, 64, 16,
            100, 4, st, st, s4, st, m, 64, 1.0, 0, None),
        "gate": lambda s4, s3, m: lib.tasft_gate_fwd(
            fake, fake, fake, fake, fake, fake, fake, None, fake, fake, None, None, fake, 1 << 20, 1,
            32, 8, 1024, 128, 64, 128, st, s4, 1, 0, None),
        "gate_target": lambda s4, s3, m: lib.tasft_gate_target_fwd(
            fake, fake, None, fake, 1, 32, 8, 1024, 128, 64, s4, st, None, 1.0, 1, 0, 1.0, 0.0, 0,
            None),
        "gate_decode_rows": lambda s4, s3, m: lib.tasft_gate_decode_rows_fwd(
            fake, fake, st, s4, fake, fake, fake, 4096, fake, fake, fake, fake, fake, fake, fake,
            fake, 1, 32, 8, 128, 128, 3, 0, 2, 0, None),
    }
    for name, call in calls.items():
        rc = call(neg, neg3, st)
        assert rc == -1 and b"non-negative" in lib.tasft_last_error(), name
    for name in ("prefill", "prefill_varlen", "decode", "decode_paged"):
        rc = calls[name](st, st3, neg)  # the mask strides
        assert rc == -1 and b"non-negative" in lib.tasft_last_error(), name
    rc = lib.tasft_mask_compact(fake, 1, 2, 4, 4, neg, 1, fake, fake, 16, fake, 1 << 20, None)
    assert rc == -1 and b"non-negative" in lib.tasft_last_error()


def test_check_raises_kernel_error_with_message():
    from tasft_amd.exceptions import KernelError
    lib = _native.load_library()
    st = _i64([0, 0, 0, 1])
    rc = lib.tasft_gate_target_fwd(None, None, None, None, 1, 1, 1, 64, 128, 64, st, st, None, 1.0, 1, 0,
                                   1.0, 0.0, 0, None)
    with pytest.raises(KernelError, match="null pointer"):
        _native.check(rc, "tasft_gate_target_fwd")


def test_gate_decode_rows_limits_are_checked_before_any_launch():
    """The one-launch decode rows take at most 8 query heads per KV head, head_dim and hidden
    up to 256 (hidden a multiple of 4) and a kept-unit stride that holds the current block;
    outside that the call returns an error without touching the GPU."""
    lib = _native.load_library()
    st = _i64([0, 0, 0, 1])
    fake = ctypes.c_void_p(16)

    def call(hq, hkv, d, hid, row, stride):
        return lib.tasft_gate_decode_rows_fwd(
            fake, fake, st, st, fake, fake, fake, stride, fake, fake, fake, fake, fake, fake, fake,
            fake, 1, hq, hkv, d, hid, row, 0, 2, 0, None)

    assert call(32, 2, 128, 128, 3, 4096) == -2 and b"8 query heads" in lib.tasft_last_error()
    assert call(32, 8, 512, 128, 3, 4096) == -2
    assert call(32, 8, 128, 260, 3, 4096) == -2
    assert call(32, 8, 128, 126, 3, 4096) == -2
    assert call(32, 8, 128, 128, 40, 4096) == -1 and b"uk_head_stride" in lib.tasft_last_error()
    assert call(32, 8, 128, 128, -1, 4096) == -1
    assert call(30, 8, 128, 128, 3, 4096) == -1 and b"multiple" in lib.tasft_last_error()
