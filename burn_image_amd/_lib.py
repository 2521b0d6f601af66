"""ctypes binding of libbiq.so (the C ABI declared in include/biq.h).

The library is built in-tree by ``python -m burn_image_amd.build``.  Loading fails loudly when it
is missing: there is no CPU or PyTorch fallback for any operator of this package.
"""
from __future__ import annotations

import ctypes
import os
import threading

PKG = os.path.dirname(os.path.abspath(__file__))
# BIQ_LIBRARY selects another build of the same ABI (e.g. a tuning variant).
LIB_PATH = os.environ.get("BIQ_LIBRARY") or os.path.join(PKG, "libbiq.so")

OK = 0
ERR_INVALID_ARG = 1
ERR_UNSUPPORTED = 2
ERR_HIP = 3

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

ROPE_INTERLEAVED = 0  # Boogu pairs (2p, 2p + 1)
ROPE_HALF = 1         # Qwen rotate_half pairs (i, i + D/2)

KEY_MASK_VALID = 0            # nonzero byte = key may be attended (Qwen attention_mask)
KEY_MASK_VALID_FILL_MEAN = 1  # as VALID; rows with no visible key = mean of V (Qwen -1e30 fill)
KEY_MASK_MASKED = 2           # nonzero byte = key masked out (Burn bool mask polarity)

Q4_NK_AXIS0 = 0  # Qwen PackedU32(0): weight [N, K], words [N, K/8], scales [N, K/blk]
Q4_KN_AXIS1 = 1  # Boogu PackedU32(1): weight [K, N], words [K/8, N], scales [K/blk, N]

# Every exported symbol with its argtypes / restype (mirrors include/biq.h).
_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
SIGNATURES = {
    "biq_version": ([], ctypes.c_char_p),
    "biq_last_error": ([], ctypes.c_char_p),
    "biq_q4_storage_block": ([_I, _I64, _I64], _I),
    "biq_q4_stored_dtype": ([_I, _I64, _I64, ctypes.c_char_p, ctypes.c_size_t], _I),
    "biq_q4_payload_layout": ([ctypes.c_char_p, _I64, _I64, _I64, ctypes.POINTER(_I), ctypes.POINTER(_I),
                               ctypes.POINTER(_I64), ctypes.POINTER(_I64)], _I),
    "biq_q4_quantize": ([_P, _P, _I, _I64, _I64, _P, _P], _I),
    "biq_q4_dequant_f32": ([_P, _P, _P, _I, _I, _I64, _I64, _P], _I),
    "biq_q4_linear": ([_P, _P, _I, _I64, _I64, _I64, _P, _P, _I, _I, _I64, _P, _P, _I], _I),
    "biq_block_glue": ([_P, _I64, _I64, _I64, _P, _P, _I, _P, _P, _P, ctypes.c_float, _P, _P, _P,
                        ctypes.c_float, _P, _P, _I], _I),
    "biq_silu": ([_P, _I64, _P, _I, _P], _I),
    "biq_release_stream_workspace": ([_P], _I),
    "biq_q4_linear_noalloc": ([_P, _P, _I, _I64, _I64, _I64, _P, _P, _I, _I, _I64, _P, _P, _I], _I),
    "biq_q4_linear_swiglu": ([_P, _P, _I, _I64, _I64, _I64, _P, _P, _P, _P, _I, _I, _I64, _P, _I], _I),
    "biq_q4_linear_qk_norm_rope": ([_P, _P, _I, _I64, _I64, _I64, _I64, _P, _P, _I, _I64, _I64, _I64,
                                    _P, _P, ctypes.c_float, ctypes.c_float, _P, _P, _I64, _I, _I,
                                    _P, _P, _P], _I),
    "biq_attention": ([_P, _P, _P, _P, _P, _I, _I, _I64, _I64, _I64, _I64, _I64, _I64,
                       ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.POINTER(_I64),
                       ctypes.POINTER(_I64), ctypes.c_float, _I, _P, _I64, _P, _I64, _I], _I),
    "biq_attention_burn": ([_P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64,
                            ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.POINTER(_I64),
                            ctypes.POINTER(_I64), _P, ctypes.POINTER(_I64), _P, _I, _I,
                            ctypes.c_float, _I, ctypes.c_float], _I),
    "biq_check_cu_seqlens": ([_P, _I64, _I64], _I),
    "biq_frame_ranges_to_cu_seqlens": ([_P, _I64, _I64, _P], _I),
    "biq_qk_norm_rope": ([_P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64,
                          ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.POINTER(_I64),
                          _P, _P, ctypes.c_float, ctypes.c_float, _P, _P, _I64, _I, _I, _P, _P, _P], _I),
}

_lib = None
_lock = threading.Lock()


class BiqError(RuntimeError):
    """A libbiq call returned an error status (the reference would panic or return Err)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[biq status {status}] {message}")
        self.status = status


class InvalidArgument(BiqError, ValueError):
    pass


class Unsupported(BiqError):
    pass


def load() -> ctypes.CDLL:
    """Load libbiq.so; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m burn_image_amd.build` "
                    "(there is no fallback implementation)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (argtypes, restype) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = lib
    return _lib


def check(status: int) -> None:
    if status == OK:
        return
    msg = load().biq_last_error().decode(errors="replace")
    if status == ERR_INVALID_ARG:
        raise InvalidArgument(status, msg)
    if status == ERR_UNSUPPORTED:
        raise Unsupported(status, msg)
    raise BiqError(status, msg)


def version() -> str:
    return load().biq_version().decode()


def strides3(values) -> ctypes.Array:
    arr = (_I64 * 3)(*[int(v) for v in values])
    return arr
