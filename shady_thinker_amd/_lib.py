"""ctypes binding of libshady_hip.so (the C ABI in include/shady_hip.h).

There is no fallback: if the library is not built, or a call fails, this
raises. The HIP kernels are the only compute path.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libshady_hip.so")
HEADER = os.path.join(ROOT, "include", "shady_hip.h")

ST_OK = 0
ST_ERR_WORKSPACE = 6
ST_F32, ST_F16, ST_BF16 = 0, 1, 2
ST_FLAG_ZEROS_PLUS_ONE = 0x1
ST_FLAG_TILED = 0x2

# st_tune (include/shady_hip.h): kernel-path overrides of one context
TUNE_KNOBS = ("DECODE_KERNEL", "STAGE_MODE", "STAGE_ROUNDS", "WAVES", "NO_COOP", "ONE_TILE", "NO_CHUNK", "NO_KSPLIT",
              "SPLIT_TILES_CU", "TOKEN_BLOCK", "I4MM_MIN_M", "I4MM_MIN_TILES", "I8MM_MIN_M", "GEMM_CB", "GEMM_NO_SPLIT",
              "STREAM_WAVES", "STREAM_TILES_WG", "STREAM_SYNC", "SPLIT_REDUCE_KERNEL", "I4MM_WAVES", "I4MM_PAIR", "I4MM_PREPASS",
              "I4MM_SPLIT_TILES")
TUNE = {name: i for i, name in enumerate(TUNE_KNOBS)}

STATUS_NAMES = {
    0: "ST_OK", 1: "ST_ERR_INVALID", 2: "ST_ERR_SHAPE", 3: "ST_ERR_ALIGN",
    4: "ST_ERR_UNSUPPORTED", 5: "ST_ERR_HIP", 6: "ST_ERR_WORKSPACE", 7: "ST_ERR_OOM",
}


class ShadyHipError(RuntimeError):
    """A C-ABI call returned a non-zero st_status (the reference panics)."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} -> {STATUS_NAMES.get(code, code)}: {message}")
        self.fn = fn
        self.code = code
        self.message = message


_P = ctypes.c_void_p
_I = ctypes.c_int
_U32 = ctypes.c_uint32
_SZ = ctypes.c_size_t

_SIGNATURES = {
    "st_last_error": (ctypes.c_char_p, []),
    "st_version": (ctypes.c_char_p, []),
    "st_context_create": (_I, [_I, ctypes.POINTER(_P)]),
    "st_context_set_stream": (_I, [_P, _P]),
    "st_context_stream": (_P, [_P]),
    "st_context_reserve_workspace": (_I, [_P, _SZ]),
    "st_context_destroy": (_I, [_P]),
    "st_context_set_tune": (_I, [_P, _I, _I]),
    "st_context_get_tune": (_I, [_P, _I, ctypes.POINTER(_I)]),
    "st_context_set_timing_events": (_I, [_P, _P, _P]),
    "st_context_pin_workspace": (_I, [_P, _I]),
    "st_alloc": (_I, [_P, _SZ, ctypes.POINTER(_P)]),
    "st_free": (_I, [_P, _P]),
    "st_upload": (_I, [_P, _P, _P, _SZ]),
    "st_write": (_I, [_P, _P, _SZ, _P, _SZ]),
    "st_read": (_I, [_P, _P, _P, _SZ]),
    "st_copy": (_I, [_P, _P, _P, _SZ]),
    "st_flush": (_I, [_P]),
    "st_gptq_i4_matvec": (_I, [_P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U32]),
    "st_gptq_i4_matvec_noalloc": (_I, [_P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U32]),
    "st_gptq_i4_silu_matvec": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U32]),
    "st_gptq_i4_gate_up_silu": (_I, [_P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U32]),
    "st_gptq_i4_dequant": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U32]),
    "st_gptq_i4_act_order": (_I, [_P, _P, _P, _P, _P, _I, _I, _I]),
    "st_gptq_i4_tiled_words": (_SZ, [_I, _I, _I]),
    "st_gptq_i4_repack": (_I, [_P, _P, _P, _I, _I, _I]),
    "st_gptq_i4_gemm": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _U32]),
    "st_gptq_i4_silu_gemm": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _U32]),
    "st_gptq_i4_gate_up_gemm": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _U32]),
    "st_bf16_matvec": (_I, [_P, _P, _I, _P, _P, _I, _I, _I]),
    "st_int8_matvec": (_I, [_P, _P, _I, _P, _P, _P, _I, _I, _I, _U32]),
    "st_int8_gemm": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _U32]),
    "st_int8_tiled_bytes": (_SZ, [_I, _I]),
    "st_int8_repack": (_I, [_P, _P, _P, _I, _I]),
}

_lib = None


def header_symbols() -> list[str]:
    """Every function the C header declares."""
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(st_\w+)\s*\(", text, re.M)


def lib() -> ctypes.CDLL:
    """Load libshady_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ShadyHipError("load", -1, f"{LIB_PATH} is not built; run `python -m shady_thinker_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, code: int) -> None:
    if code != ST_OK:
        raise ShadyHipError(fn, code, lib().st_last_error().decode())


def call(fn: str, *args) -> None:
    check(fn, getattr(lib(), fn)(*args))
