"""ctypes binding of the gfx950 C-ABI library ``libtasft_amd.so``.

The library is built in-tree by ``python -m tasft_amd.csrc.build`` (or
``__graft_entry__.build()``). There is no fallback: if the library is missing or fails
to load, every kernel entry point raises ``KernelError``.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

from tasft_amd.exceptions import KernelError

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libtasft_amd.so"

# Every symbol the header include/tasft_amd.h declares.
DECODE_NOALLOC_MAX_BYTES = 16 << 20  # TASFT_DECODE_NOALLOC_MAX_BYTES
EXPORTED_SYMBOLS = (
    "tasft_last_error",
    "tasft_abi_version",
    "tasft_bsfa_prefill_workspace_bytes",
    "tasft_bsfa_prefill_fwd",
    "tasft_bsfa_prefill_varlen_fwd",
    "tasft_bsfa_varlen_zero_tail",
    "tasft_bsfa_decode_workspace_bytes",
    "tasft_bsfa_decode_fwd",
    "tasft_bsfa_decode_paged_fwd",
    "tasft_bsfa_decode_fwd_noalloc",
    "tasft_gate_workspace_bytes",
    "tasft_gate_fwd",
    "tasft_gate_debug_wait_fault",
    "tasft_gate_rows_fwd",
    "tasft_gate_decode_rows_fwd",
    "tasft_gate_bwd_workspace_bytes",
    "tasft_gate_bwd",
    "tasft_gate_target_fwd",
    "tasft_gate_kl_fwd",
    "tasft_mask_compact_workspace_bytes",
    "tasft_mask_compact",
    "tasft_mask_from_indices",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I64P = ctypes.POINTER(ctypes.c_int64)
_F = ctypes.c_float
_I = ctypes.c_int
_SZ = ctypes.c_size_t

_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "tasft_last_error": (ctypes.c_char_p, []),
    "tasft_abi_version": (_I, []),
    "tasft_gate_debug_wait_fault": (_I, [_I]),
    "tasft_bsfa_prefill_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "tasft_bsfa_prefill_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64P, _I64P, _I64P, _I64P, _I64P, _F, _I, _I, _P],
    ),
    "tasft_bsfa_prefill_varlen_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64P, _I64P, _I64P, _I64P, _I64P, _F, _I, _I, _P],
    ),
    "tasft_bsfa_varlen_zero_tail": (_I, [_P, _P, _I64, _I64, _I64, _I64, _I64P, _P]),
    "tasft_bsfa_decode_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "tasft_bsfa_decode_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64P, _I64P, _I64P, _I64P, _I64P, _F, _I, _P],
    ),
    "tasft_bsfa_decode_paged_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64, _I64P, _I64P, _I64P, _I64P, _I64P, _I64, _F, _I, _P],
    ),
    "tasft_bsfa_decode_fwd_noalloc": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64P, _I64P, _I64P, _I64P, _I64P, _F, _I, _P],
    ),
    "tasft_gate_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I64]),
    "tasft_gate_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64,
         _I64, _I64, _I64P, _I64P, _I, _I, _P],
    ),
    "tasft_gate_rows_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P],
    ),
    "tasft_gate_decode_rows_fwd": (
        _I,
        [_P, _P, _I64P, _I64P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
         _I64, _I64, _I64, _I64, _I, _I, _I, _P],
    ),
    "tasft_gate_bwd_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "tasft_gate_bwd": (
        _I,
        [_P, _P, _P, _SZ, _P, _SZ, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P],
    ),
    "tasft_gate_kl_fwd": (_I, [_P, _P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "tasft_gate_target_fwd": (
        _I,
        [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _I64P, _F, _I, _I,
         _F, _F, _I, _P],
    ),
    "tasft_mask_compact_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "tasft_mask_compact": (
        _I,
        [_P, _I64, _I64, _I64, _I64, _I64P, _I, _P, _P, _I64, _P, _SZ, _P],
    ),
    "tasft_mask_from_indices": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P]),
}


def load_library() -> ctypes.CDLL:
    """Load (once) and return the C-ABI library; raises ``KernelError`` if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise KernelError(
                f"HIP library not built: {LIB_PATH} is missing "
                "(run `python -m tasft_amd.csrc.build`)",
                context={"path": str(LIB_PATH)},
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:
            raise KernelError(f"failed to load {LIB_PATH}: {exc}", context={"path": str(LIB_PATH)}) from exc
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def is_available() -> bool:
    """True if the library loads (does not touch the GPU)."""
    try:
        load_library()
    except KernelError:
        return False
    return True


def strides(t: torch.Tensor) -> ctypes.Array:
    """Element strides of a tensor as a C int64 array."""
    return (ctypes.c_int64 * t.dim())(*t.stride())


def strides_array(values) -> ctypes.Array:
    """A list of element strides as a C int64 array."""
    return (ctypes.c_int64 * len(values))(*values)


# Element types of the 16-bit tensors (TASFT_DTYPE_BF16 / TASFT_DTYPE_F16).
DTYPE_BF16 = 0
DTYPE_F16 = 1
_DTYPE_CODES = {torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}
KERNEL_DTYPES = tuple(_DTYPE_CODES)


def dtype_code(dtype: torch.dtype, what: str) -> int:
    """The C-ABI ``dtype`` argument for a torch dtype; raises ``KernelError`` for any other
    than bf16 / fp16."""
    code = _DTYPE_CODES.get(dtype)
    if code is None:
        raise KernelError(f"{what}: the HIP kernels take bf16 or fp16 tensors, got {dtype}",
                          context={"dtype": str(dtype)})
    return code


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def check(status: int, what: str, context: dict[str, object] | None = None) -> None:
    """Raise ``KernelError`` with the library's message when ``status`` is non-zero."""
    if status != 0:
        msg = load_library().tasft_last_error().decode(errors="replace")
        raise KernelError(f"{what} failed ({status}): {msg}", context={"status": status, **(context or {})})


__all__ = ["DTYPE_BF16", "DTYPE_F16", "EXPORTED_SYMBOLS", "KERNEL_DTYPES", "LIB_PATH", "check",
           "dtype_code", "is_available", "load_library", "ptr", "stream_handle", "strides",
           "strides_array"]
