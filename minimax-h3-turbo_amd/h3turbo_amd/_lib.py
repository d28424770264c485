"""ctypes binding of the h3k C ABI (include/h3k.h).  The library must be built in-tree first:

    python minimax-h3-turbo_amd/build_lib.py

Loading fails loudly when it is missing: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libh3k.so")

# element type codes, quant modes and error codes of h3k.h
BF16, F16, F32, FP8E4M3 = 0, 1, 2, 3
MODE = {"ck": 0, "eager": 1}
EINVAL, ELAUNCH, ESPACE = -1, -2, -3

_i64, _int, _ptr, _size = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t

SIGNATURES = {
    "h3k_version": (_int, []),
    "h3k_last_error": (ctypes.c_char_p, []),
    "h3k_rotate_quant": (_int, [_ptr, _int, _i64, _i64, _i64, _int, _int, _ptr, _i64, _ptr, _ptr]),
    "h3k_rotate": (_int, [_ptr, _int, _i64, _i64, _i64, _int, _ptr, _i64, _ptr]),
    "h3k_decode_w4": (_int, [_ptr, _i64, _ptr, _int, _i64, _ptr, _i64, _i64, _int, _ptr, _i64, _ptr]),
    "h3k_gemm_a8w8": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _int, _ptr, _int, _i64, _ptr, _ptr]),
    "h3k_rotate_quant_act": (_int, [_ptr, _int, _i64, _i64, _i64, _int, _int, _int, _ptr, _i64, _ptr, _ptr]),
    "h3k_gemm_w4a8_workspace": (_i64, [_i64, _i64, _i64]),
    "h3k_gemm_w4a8": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _ptr, _int, _i64, _ptr, _int, _ptr, _ptr, _i64, _i64, _i64,
                             _int, _ptr, _int, _i64, _ptr, _ptr, _ptr]),
    "h3k_w4a8_linear_workspace": (_size, [_i64, _i64, _i64]),
    "h3k_w4a8_linear_noalloc": (_int, [_ptr, _int, _i64, _i64, _i64, _ptr, _i64, _ptr, _int, _i64, _ptr, _ptr, _i64, _int,
                                       _int, _ptr, _int, _ptr, _int, _i64, _ptr]),
    "h3k_w4a8_linear": (_int, [_ptr, _int, _i64, _i64, _i64, _ptr, _i64, _ptr, _int, _i64, _ptr, _ptr, _i64, _int, _int,
                               _ptr, _int, _ptr, _int, _i64, _ptr, _size, _ptr]),
    "h3k_copy_h2d_async": (_int, [_ptr, _ptr, _size, _ptr]),
    "h3k_gated_add": (_int, [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64, _i64, _int, _ptr]),
    "h3k_gated_add_rms_modulate": (_int, [_ptr, _i64, _ptr, _i64, _ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _i64, _ptr,
                                          ctypes.c_float, _ptr, _i64, _int, _ptr]),
    "h3k_gemm_a16": (_int, [_ptr, _int, _i64, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _ptr, _int, _i64, _ptr]),
    "h3k_w8_packed_bytes": (_i64, [_i64, _i64]),
    "h3k_decode_w4_packed": (_int, [_ptr, _i64, _ptr, _int, _i64, _ptr, _i64, _i64, _int, _ptr, _ptr]),
    "h3k_pack_w8": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr]),
    "h3k_gemm_packed_serves": (_int, [_i64, _i64, _i64]),
    "h3k_gemm_packed_split_bytes": (_i64, [_i64, _i64, _i64]),
    "h3k_gemm_a8w8_packed_ws": (_int, [_ptr, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _int, _ptr, _int, _i64, _ptr,
                                       _size, _ptr]),
    "h3k_gemm_a8w8_packed": (_int, [_ptr, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _int, _ptr, _int, _i64, _ptr,
                                    _ptr]),
    "h3k_qk_norm_rope": (_int, [_ptr, _i64, _ptr, _i64, _i64, _int, _int, _ptr, _ptr, _ptr, _ptr, _i64, _int,
                                ctypes.c_float, _ptr]),
    "h3k_qkv_split_norm_rope": (_int, [_ptr, _i64, _i64, _int, _int, _ptr, _ptr, _ptr, _ptr, _i64, _int, ctypes.c_float,
                                       _ptr, _ptr, _ptr, _i64, _ptr]),
    "h3k_rotate_quant_heads": (_int, [_ptr, _int, _i64, _i64, _i64, _int, _i64, _int, _int, _ptr, _i64, _ptr, _ptr]),
    "h3k_rms_modulate": (_int, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _i64, _ptr, ctypes.c_float, _ptr, _i64, _int,
                                _ptr]),
}
ABI_VERSION = 7

_LIB: Optional[ctypes.CDLL] = None
_LOCK = threading.Lock()


def load() -> ctypes.CDLL:
    """The loaded library (cached).  RuntimeError when it has not been built."""
    global _LIB
    if _LIB is None:
        with _LOCK:
            if _LIB is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(f"h3k HIP library not found at {LIB_PATH}; build it with "
                                       "`python minimax-h3-turbo_amd/build_lib.py` (hipcc, gfx950)")
                lib = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(lib, name)
                    fn.restype, fn.argtypes = res, args
                if lib.h3k_version() != ABI_VERSION:
                    raise RuntimeError(f"{LIB_PATH} has ABI {lib.h3k_version()}, expected {ABI_VERSION}: rebuild it")
                _LIB = lib
    return _LIB


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    msg = (load().h3k_last_error() or b"").decode(errors="replace")
    if rc == EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_ACT_CODE = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}
_SCALE_CODE = {torch.float8_e4m3fn: FP8E4M3, torch.uint8: FP8E4M3, torch.float16: F16, torch.bfloat16: BF16,
               torch.float32: F32}


def act_code(dt: torch.dtype) -> int:
    try:
        return _ACT_CODE[dt]
    except KeyError:
        raise ValueError(f"the HIP path takes bf16, f16 or f32 activations/outputs, got {dt}") from None


def scale_code(dt: torch.dtype) -> int:
    try:
        return _SCALE_CODE[dt]
    except KeyError:
        raise ValueError(f"s_rel dtype {dt} unsupported (float8_e4m3fn/uint8 bytes, float16, bfloat16, float32)") from None
