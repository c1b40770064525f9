"""CPU oracle for the quantized-linear hot path (ctypes wrapper over oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker (or the timed CPU
baseline), never as the product path. The shipped package never imports it.

Every function restates reference behaviour; the C source cites the
reference file:line for each. See oracle.c's header for what pins each
function.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_D = ctypes.c_double


def build(force: bool = False) -> str:
    """Compile oracle.c with gcc (make). Returns the library path."""
    src = os.path.join(_HERE, "oracle.c")
    if force or not os.path.exists(_LIB_PATH) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        sigs = {
            "orc_rng_draws": (_U64, [_U64, _P, _I64]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_gen_normal_f32": (None, [_U64, _P, _I64, _D, _D]),
            "orc_gen_normal_f16": (None, [_U64, _P, _I64, _D, _D]),
            "orc_gen_abs_normal_f16": (None, [_U64, _P, _I64, _D]),
            "orc_gen_abs_normal_f32": (None, [_U64, _P, _I64, _D]),
            "orc_gen_nibbles": (None, [_U64, _P, _I64, _I, _I]),
            "orc_gen_int8": (None, [_U64, _P, _I64, _I, _I]),
            "orc_gen_perm": (None, [_U64, _P, ctypes.c_int32]),
            "orc_dequant_i4": (ctypes.c_float, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint16]),
            "orc_gptq_dequant_f32": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
            "orc_gptq_dequant_bf16": (None, [_P, _P, _I, _I, _I, _P]),
            "orc_gptq_matvec_wgsl": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I]),
            "orc_fused_silu_gptq_wgsl": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
            "orc_gate_up_silu_wgsl": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
            "orc_gptq_matvec_f64": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
            "orc_silu_mul_f64": (None, [_P, _P, _P, _I64]),
            "orc_silu_gate_f64": (None, [_P, _P, _P, _I64]),
            "orc_int8_matvec_f64": (None, [_P, _P, _P, _I, _I, _I, _P]),
            "orc_gptq_matvec_4t_omp": (_I, [_P, _P, _P, _P, _I, _I, _I, _I]),
            "orc_bf16_matvec_wgsl": (None, [_P, _P, _P, _I, _I, _I]),
            "orc_bf16_matvec_f64": (None, [_P, _P, _I, _I, _I, _P]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------- generators
def rng_draws(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().orc_rng_draws(seed, _p(out), n)
    return out


def normal_f32(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, np.float32)
    lib().orc_gen_normal_f32(seed, _p(out), n, mean, std)
    return out


def normal_f16(seed, n, mean=0.0, std=1.0):
    out = np.empty(n, np.uint16)
    lib().orc_gen_normal_f16(seed, _p(out), n, mean, std)
    return out.view(np.float16)


def abs_normal_f16(seed, n, std):
    out = np.empty(n, np.uint16)
    lib().orc_gen_abs_normal_f16(seed, _p(out), n, std)
    return out.view(np.float16)


def abs_normal_f32(seed, n, std):
    out = np.empty(n, np.float32)
    lib().orc_gen_abs_normal_f32(seed, _p(out), n, std)
    return out


def nibbles(seed, nwords, lo=0, hi=15):
    out = np.empty(nwords, np.uint32)
    lib().orc_gen_nibbles(seed, _p(out), nwords, lo, hi)
    return out


def int8(seed, n, lo=-127, hi=127):
    out = np.empty(n, np.int8)
    lib().orc_gen_int8(seed, _p(out), n, lo, hi)
    return out


def perm(seed, n):
    out = np.empty(n, np.int32)
    lib().orc_gen_perm(seed, _p(out), n)
    return out


# --------------------------------------------------------------- scalars
def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(x)


def f32_to_bf16(x: float) -> int:
    return lib().orc_f32_to_bf16(x)


def dequant_i4(q: int, z: int, scale_bits: int) -> float:
    return lib().orc_dequant_i4(q, z, scale_bits)


# --------------------------------------------------------------- tensors
def gptq_dequant_f32(qweight, scales, K, N, gs, qzeros=None, g_idx=None, zero_offset=0):
    qw = _c(qweight, np.uint32)
    sc = _c(np.asarray(scales).view(np.uint16), np.uint16)
    qz = _c(qzeros, np.uint32)
    gi = _c(g_idx, np.int32)
    out = np.empty((K, N), np.float32)
    lib().orc_gptq_dequant_f32(_p(qw), _p(sc), _p(qz), _p(gi), K, N, gs, zero_offset, _p(out))
    return out


def gptq_dequant_bf16(qweight, scales, K, N, gs):
    qw = _c(qweight, np.uint32)
    sc = _c(np.asarray(scales).view(np.uint16), np.uint16)
    out = np.empty((K, N), np.uint16)
    lib().orc_gptq_dequant_bf16(_p(qw), _p(sc), K, N, gs, _p(out))
    return out


def gptq_matvec_wgsl(x, qweight, scales, K, N, gs, variant=1, contract=1):
    xx = _c(x, np.float32)
    qw = _c(qweight, np.uint32)
    sc = _c(np.asarray(scales).view(np.uint16), np.uint16)
    y = np.empty(N, np.float32)
    lib().orc_gptq_matvec_wgsl(_p(xx), _p(qw), _p(sc), _p(y), K, N, gs, variant, contract)
    return y


def fused_silu_gptq_wgsl(a, b, qweight, scales, K, N, gs, variant=1, contract=1):
    aa, bb = _c(a, np.float32), _c(b, np.float32)
    qw = _c(qweight, np.uint32)
    sc = _c(np.asarray(scales).view(np.uint16), np.uint16)
    y = np.empty(N, np.float32)
    lib().orc_fused_silu_gptq_wgsl(_p(aa), _p(bb), _p(qw), _p(sc), _p(y), K, N, gs, variant, contract)
    return y


def gate_up_silu_wgsl(x, qg, sg, qu, su, K, N, gs, variant=1, contract=1):
    xx = _c(x, np.float32)
    qg_, qu_ = _c(qg, np.uint32), _c(qu, np.uint32)
    sg_ = _c(np.asarray(sg).view(np.uint16), np.uint16)
    su_ = _c(np.asarray(su).view(np.uint16), np.uint16)
    y = np.empty(N, np.float32)
    lib().orc_gate_up_silu_wgsl(_p(xx), _p(qg_), _p(sg_), _p(qu_), _p(su_), _p(y), K, N, gs, variant, contract)
    return y


def gptq_matvec_f64(x, qweight, scales, K, N, gs, qzeros=None, g_idx=None, zero_offset=0):
    """x: [M, K] or [K] (any float dtype, converted exactly to f64)."""
    xx = np.asarray(x)
    M = 1 if xx.ndim == 1 else xx.shape[0]
    xd = _c(xx.reshape(M, K), np.float64)
    qw = _c(qweight, np.uint32)
    sc = _c(np.asarray(scales).view(np.uint16), np.uint16)
    qz = _c(qzeros, np.uint32)
    gi = _c(g_idx, np.int32)
    y = np.empty((M, N), np.float64)
    lib().orc_gptq_matvec_f64(_p(xd), _p(qw), _p(sc), _p(qz), _p(gi), M, K, N, gs, zero_offset, _p(y))
    return y if xx.ndim > 1 else y[0]


def silu_mul_f64(a, b):
    aa, bb = _c(a, np.float32), _c(b, np.float32)
    out = np.empty(aa.shape, np.float64)
    lib().orc_silu_mul_f64(_p(aa), _p(bb), _p(out), aa.size)
    return out


def silu_gate_f64(g, u):
    gg, uu = _c(g, np.float64), _c(u, np.float64)
    out = np.empty(gg.shape, np.float64)
    lib().orc_silu_gate_f64(_p(gg), _p(uu), _p(out), gg.size)
    return out


def int8_matvec_f64(x, w, scale, K, N):
    """x: [M, K] or [K]; w: int8 [N, K]; scale: f32 [N]."""
    xx = np.asarray(x)
    M = 1 if xx.ndim == 1 else xx.shape[0]
    xd = _c(xx.reshape(M, K), np.float64)
    ww = _c(w, np.int8)
    ss = _c(scale, np.float32)
    y = np.empty((M, N), np.float64)
    lib().orc_int8_matvec_f64(_p(xd), _p(ww), _p(ss), M, K, N, _p(y))
    return y if xx.ndim > 1 else y[0]


def bf16_matvec_wgsl(x, w, K, N, contract=1):
    """bf16_matvec.wgsl order: x f32 [K], w bf16 bits uint16 [N, K] -> f32 [N]."""
    xx = _c(x, np.float32)
    ww = _c(w, np.uint16)
    y = np.empty(N, np.float32)
    lib().orc_bf16_matvec_wgsl(_p(xx), _p(ww), _p(y), K, N, contract)
    return y


def bf16_matvec_f64(x, w, K, N):
    """x: [M, K] or [K] (any float dtype); w: bf16 bits uint16 [N, K]."""
    xx = np.asarray(x)
    M = 1 if xx.ndim == 1 else xx.shape[0]
    xd = _c(xx.reshape(M, K), np.float64)
    ww = _c(w, np.uint16)
    y = np.empty((M, N), np.float64)
    lib().orc_bf16_matvec_f64(_p(xd), _p(ww), M, K, N, _p(y))
    return y if xx.ndim > 1 else y[0]


def bf16_case(seed: int, K: int, N: int, M: int = 1, std=0.02):
    """Seeded bf16 weight [N, K] ~N(0, std) (RNE to bf16) and f32 x ~N(0,1) [M, K]."""
    base = seed * 16
    wf = normal_f32(base + 1, N * K, 0.0, std)
    w = np.array([f32_to_bf16(float(v)) for v in wf], np.uint16) if N * K <= 4096 else _bf16_bits(wf)
    return {"K": K, "N": N, "w": w.reshape(N, K), "x": normal_f32(base + 5, M * K).reshape(M, K)}


def _bf16_bits(f32: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (finite inputs), vectorised."""
    u = np.ascontiguousarray(f32, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def gptq_matvec_4t_omp(x, qweight, scales, K, N, gs, threads=0):
    """Timed CPU baseline: WGSL-order gptq_matvec_4t on `threads` cores.
    Returns (y, threads_used)."""
    xx = _c(x, np.float32)
    qw = _c(qweight, np.uint32)
    sc = _c(np.asarray(scales).view(np.uint16), np.uint16)
    y = np.empty(N, np.float32)
    used = lib().orc_gptq_matvec_4t_omp(_p(xx), _p(qw), _p(sc), _p(y), K, N, gs, threads)
    return y, used


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b.ravel())
    num = np.linalg.norm((a - b).ravel())
    return float(num / den) if den > 0 else float(num)


# ------------------------------------------------ standard synthetic inputs
def gptq_case(seed: int, K: int, N: int, gs: int = 128, zeros: bool = False,
              act_order: bool = False, M: int = 0, x_dtype=np.float32, scale_std=0.02):
    """Seeded GPTQ int4 case with per-tensor sub-seeds seed*16 + {1..6}.

    qweight u32[K/8, N] (nibbles uniform 0..15), scales f16[G, N] ~|N(0,
    scale_std)|, qzeros u32[G, N/8] uniform 0..15 (or None), g_idx =
    perm[k] // gs for a seeded Fisher-Yates perm (or None), x ~N(0,1) of
    shape [K] (M == 0) or [M, K].
    """
    G = K // gs
    base = seed * 16
    case = {
        "K": K, "N": N, "gs": gs,
        "qweight": nibbles(base + 1, (K // 8) * N).reshape(K // 8, N),
        "scales": abs_normal_f16(base + 2, G * N, scale_std).reshape(G, N),
        "qzeros": nibbles(base + 3, G * (N // 8)).reshape(G, N // 8) if zeros else None,
        "g_idx": (perm(base + 4, K) // gs).astype(np.int32) if act_order else None,
    }
    n_x = K if M == 0 else M * K
    if x_dtype == np.float16:
        x = normal_f16(base + 5, n_x)
    else:
        x = normal_f32(base + 5, n_x)
    case["x"] = x if M == 0 else x.reshape(M, K)
    return case


def int8_case(seed: int, K: int, N: int, M: int = 1, x_dtype=np.float16):
    base = seed * 16
    n_x = M * K
    x = normal_f16(base + 5, n_x) if x_dtype == np.float16 else normal_f32(base + 5, n_x)
    return {
        "K": K, "N": N, "M": M,
        "w": int8(base + 1, N * K).reshape(N, K),
        "scale": abs_normal_f32(base + 2, N, 0.01),
        "x": x.reshape(M, K),
    }
