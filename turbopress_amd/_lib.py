"""ctypes binding of libturbopress_amd.so (the C ABI in include/turbopress_amd.h).

The library is loaded from the package directory.  When it is missing or
fails to load, ``lib()`` raises: the package has no CPU fallback for any
operation on the packed path.
"""

from __future__ import annotations

import ctypes
from ctypes import c_int, c_int64, c_void_p, c_char_p, POINTER, c_uint8
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libturbopress_amd.so"
ABI_VERSION = 1

TP_OK = 0
TP_ERR_NULL_POINTER = 1
TP_ERR_UNSUPPORTED_BITS = 2
TP_ERR_UNSUPPORTED_STATES = 3
TP_ERR_BAD_DIMS = 4
TP_ERR_MISALIGNED = 5
TP_ERR_BAD_BLOCK = 6
TP_ERR_HIP = 7
TP_ERR_WORKSPACE = 8
TP_ERR_BAD_LAYOUT = 9

# Every exported symbol with its (restype, argtypes).
_P = c_void_p
_I64 = c_int64
SIGNATURES: dict[str, tuple] = {
    "tp_abi_version": (c_int, []),
    "tp_status_string": (c_char_p, [c_int]),
    "tp_subset_lut": (c_int, [c_int, POINTER(c_uint8), c_int]),
    "tp_read_probe": (c_int, [_P, _I64, _P, _P]),
    "tp_viterbi_workspace_bytes": (_I64, [_I64, _I64]),
    "tp_tcq_viterbi": (c_int, [_P, _I64, _I64, _I64, _P, c_int, c_int, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "tp_fwht_scale": (c_int, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "tp_block_fwht_rows": (c_int, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "tp_window_decode_levels": (c_int, [_P, _I64, _P, _I64, _I64, _I64, c_int, c_int, _P, _I64, _P]),
    "tp_decode_rows": (c_int, [_P, _I64, _P, _I64, _P, _P, _I64, _I64, c_int, c_int, _P, _I64, _P]),
    "tp_tcq_gemv": (c_int, [_P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, c_int, c_int, _P, _P]),
    "tp_fwht_scale_padded": (c_int, [_P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "tp_tiled_layout": (c_int, [_I64, _I64, c_int, POINTER(c_int64), POINTER(c_int64),
                                POINTER(c_int64), POINTER(c_int64), POINTER(c_int64)]),
    "tp_retile": (c_int, [_P, _I64, _P, _I64, _I64, _I64, c_int, _P, _P, _P]),
    "tp_gemv_workspace_bytes": (c_int64, [_I64, _I64]),
    "tp_linear_forward_plan": (c_int, [POINTER(c_int64), c_int, _I64, _I64, c_int, _I64, _I64, c_int, _I64,
                                       POINTER(c_int64)]),
    "tp_tcq_gemv_tiled": (c_int, [_P, _I64, _I64, _P, _P, _P, _P, _P, _I64, _I64, c_int, c_int,
                                  _P, _I64, _P, _I64, _P]),
    "tp_decode_tiled": (c_int, [_P, _P, _P, _P, _I64, _I64, c_int, c_int, _P, _I64, _P]),
    "tp_packed_linear_forward": (c_int, [_P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64,
                                         c_int, c_int, _P, _I64, _P, _I64, _P]),
    "tp_packed_linear_forward_noalloc": (c_int, [_P, _I64, _I64, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64,
                                                 c_int, c_int, _P, _I64, _P]),
    "tp_packed_linear_forward_group": (c_int, [c_int, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P,
                                               _I64, c_int, c_int, _P, _P, _P, _P, _P]),
}

class StackLinear(ctypes.Structure):
    """tp_stack_linear (include/turbopress_amd.h)."""
    _fields_ = [
        ("path_tiled", c_void_p), ("member_tiled", c_void_p),
        ("x", c_void_p), ("ldx", c_int64), ("rot_scale", c_void_p), ("block", c_int64),
        ("scales", c_void_p), ("bias", c_void_p), ("y", c_void_p), ("ldy", c_int64),
        ("n", c_int64), ("d", c_int64), ("phase", ctypes.c_int32), ("reserved", ctypes.c_int32),
    ]


SIGNATURES.update({
    "tp_stack_plan_bytes": (c_int64, [POINTER(StackLinear), c_int, c_int, _I64]),
    "tp_stack_plan_init": (c_int, [POINTER(StackLinear), c_int, c_int, _I64, _P, _I64]),
    "tp_stack_run": (c_int, [_P, _I64, _P, c_int, c_int, c_int, _I64, _P]),
    "tp_stack_rotate": (c_int, [_P, _I64, _P]),
    "tp_stack_gemv": (c_int, [_P, _I64, _P, c_int, c_int, c_int, _I64, _P]),
    "tp_stack_plan_blocks": (c_int64, [POINTER(c_int64), c_int]),
    "tp_stack_error": (c_int, [_P, POINTER(c_int)]),
})

_LIB: ctypes.CDLL | None = None
_LOAD_ERROR: str | None = None


class TurboPressError(RuntimeError):
    """A C-ABI call returned a HIP/runtime failure status."""


def _load() -> ctypes.CDLL:
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        _LOAD_ERROR = (f"{LIB_PATH.name} is not built; run `python -m turbopress_amd.build` "
                       "(turbopress_amd has no CPU fallback)")
        raise RuntimeError(_LOAD_ERROR)
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.tp_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH.name} ABI version {ver}, expected {ABI_VERSION}; rebuild")
    _LIB = lib
    return lib


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError when it is unavailable."""
    return _load()


def available() -> bool:
    try:
        _load()
        return True
    except (RuntimeError, OSError):
        return False


def status_string(status: int) -> str:
    return lib().tp_status_string(status).decode()


def check(status: int, what: str) -> None:
    """Map a C-ABI status to the reference's exception types: argument
    problems raise ValueError (runtime.py:222-225, 305-306), runtime failures
    raise TurboPressError (a RuntimeError)."""
    if status == TP_OK:
        return
    msg = f"{what}: {status_string(status)} (status {status})"
    if status in (TP_ERR_HIP, TP_ERR_WORKSPACE):
        raise TurboPressError(msg)
    raise ValueError(msg)
