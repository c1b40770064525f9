"""Linear-layer dispatch helpers, mirroring the reference's `Model` helpers.

`gptq_matvec` and `fused_silu_gptq_down` keep the argument order and meaning
of src/model.rs:357-361 and :383-388 (gpu, [name,] input buffers, weight
buffers, output, k, n); the group size comes from QuantConfig as in
src/model.rs:366. Instead of writing a uniform and calling
GpuContext::dispatch with a WGSL shader (src/model.rs:348-381), each helper
calls one C-ABI entry point of libshady_hip. Errors raise ShadyHipError
(the reference panics).

All tensors are torch device tensors: x/a/b/output f32 (x may be f16),
qweight int32 [K/8, N], scales f16 [K/gs, N], optional qzeros int32
[K/gs, N/8], optional perm int32 [K].
"""
from __future__ import annotations

from ._lib import ST_F16, ST_F32, ST_FLAG_TILED, call, lib
from .gpu import ptr
from .weights import GptqWeight, Int8Weight


def _xdtype(t) -> int:
    import torch

    if t.dtype == torch.float32:
        return ST_F32
    if t.dtype == torch.float16:
        return ST_F16
    raise TypeError(f"activation dtype {t.dtype} (need float32 or float16)")


def _rows(t, k: int) -> int:
    if t.numel() % k or t.numel() == 0:
        raise ValueError(f"input of {t.numel()} elements is not [M, {k}] with M >= 1")
    return t.numel() // k


# Argument checks the C ABI cannot make: it receives bare pointers, so a
# wrong dtype or a short buffer would be read or written past its end on the
# device. Every helper checks its tensors here before the call.
def _need(t, name: str, dtypes, numel: int) -> None:
    if t is None:
        raise ValueError(f"{name} is required")
    if t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype} (need {' or '.join(str(d) for d in dtypes)})")
    if not t.is_contiguous():
        raise ValueError(f"{name}: not contiguous")
    if t.numel() < numel:
        raise ValueError(f"{name}: {t.numel()} elements, need at least {numel}")


def _torch():
    import torch

    return torch


def _check_gptq(qweight, scales, qzeros, perm, k: int, n: int, group_size: int, flags: int) -> None:
    torch = _torch()
    if group_size <= 0 or k <= 0 or n <= 0 or k % group_size or k % 8 or n % 8:
        raise ValueError(f"GPTQ weight {k} x {n}, group size {group_size}: K and N multiples of 8, K of the group")
    words = lib().st_gptq_i4_tiled_words(k, n, group_size) if flags & ST_FLAG_TILED else k // 8 * n
    _need(qweight, "qweight", (torch.int32,), words)
    _need(scales, "scales", (torch.float16,), k // group_size * n)
    if qzeros is not None:
        _need(qzeros, "qzeros", (torch.int32,), k // group_size * (n // 8))
    if perm is not None:
        _need(perm, "perm", (torch.int32,), k)


def _check_io(x, k: int, out, n: int, x_dtypes=None, out_dtypes=None, name: str = "input") -> int:
    torch = _torch()
    _need(x, name, x_dtypes or (torch.float32, torch.float16), 0)
    m = _rows(x, k)
    _need(out, "output", out_dtypes or (torch.float32,), m * n)
    return m


def gptq_matvec(gpu, name: str, input, qweight, scales, output, k: int, n: int, group_size: int = 128,
                qzeros=None, perm=None, flags: int = 0) -> None:
    """output[M, n] = input[M, k] . dequant(W)  (src/model.rs:357-381)."""
    _check_gptq(qweight, scales, qzeros, perm, k, n, group_size, flags)
    m = _check_io(input, k, output, n)
    gpu.sync_stream()
    call("st_gptq_i4_matvec", gpu.handle, ptr(input), _xdtype(input), ptr(qweight), ptr(scales), ptr(qzeros),
         ptr(perm), ptr(output), m, k, n, group_size, flags)


def fused_silu_gptq_down(gpu, gate_out, up_out, down_qw, down_sc, output, k: int, n: int, group_size: int = 128,
                         qzeros=None, perm=None, flags: int = 0) -> None:
    """output = (silu(gate_out) * up_out) . dequant(W_down)  (src/model.rs:383-408)."""
    torch = _torch()
    _check_gptq(down_qw, down_sc, qzeros, perm, k, n, group_size, flags)
    m = _check_io(gate_out, k, output, n, x_dtypes=(torch.float32,), name="gate_out")
    _need(up_out, "up_out", (torch.float32,), m * k)
    gpu.sync_stream()
    call("st_gptq_i4_silu_matvec", gpu.handle, ptr(gate_out), ptr(up_out), ptr(down_qw), ptr(down_sc),
         ptr(qzeros), ptr(perm), ptr(output), m, k, n, group_size, flags)


def fused_gate_up_silu(gpu, input, gate_qw, gate_sc, up_qw, up_sc, output, k: int, n: int, group_size: int = 128,
                       gate_qz=None, up_qz=None, perm=None, flags: int = 0) -> None:
    """output = silu(input . Wg) * (input . Wu)  (fused_gate_up_silu_4t.wgsl)."""
    _check_gptq(gate_qw, gate_sc, gate_qz, perm, k, n, group_size, flags)
    _check_gptq(up_qw, up_sc, up_qz, perm, k, n, group_size, flags)
    m = _check_io(input, k, output, n)
    gpu.sync_stream()
    call("st_gptq_i4_gate_up_silu", gpu.handle, ptr(input), _xdtype(input), ptr(gate_qw), ptr(gate_sc),
         ptr(gate_qz), ptr(up_qw), ptr(up_sc), ptr(up_qz), ptr(perm), ptr(output), m, k, n, group_size, flags)


def gptq_dequant(gpu, qweight, scales, out, k: int, n: int, group_size: int = 128, qzeros=None, g_idx=None,
                 flags: int = 0) -> None:
    """out[k, n] = dequant(W) in out's dtype (float32 exact, bfloat16 RNE as
    src/weights.rs:257-313)."""
    import torch

    od = {torch.float32: 0, torch.bfloat16: 2}.get(out.dtype)
    if od is None:
        raise TypeError(f"dequant output dtype {out.dtype}")
    if g_idx is not None:
        _need(g_idx, "g_idx", (torch.int32,), k)
    _check_gptq(qweight, scales, qzeros, None, k, n, group_size, flags)
    _need(out, "out", (out.dtype,), k * n)
    gpu.sync_stream()
    call("st_gptq_i4_dequant", gpu.handle, ptr(qweight), ptr(scales), ptr(qzeros), ptr(g_idx), ptr(out), od, k, n,
         group_size, flags)


def int8_matvec(gpu, x, w, scale, y, k: int, n: int, flags: int = 0) -> None:
    """y[M, n] = x[M, k] . (w[n, k]^T * scale[n]) (INT8 per-channel); flags
    ST_FLAG_TILED when w is in the layout of st_int8_repack."""
    torch = _torch()
    m = _check_io(x, k, y, n)
    nbytes = lib().st_int8_tiled_bytes(k, n) if flags & ST_FLAG_TILED else k * n
    _need(w, "w", (torch.int8,), nbytes)
    _need(scale, "scale", (torch.float32,), n)
    gpu.sync_stream()
    call("st_int8_matvec", gpu.handle, ptr(x), _xdtype(x), ptr(w), ptr(scale), ptr(y), m, k, n, flags)


def int8_gemm(gpu, a, w, scale, c, k: int, n: int, flags: int = 0) -> None:
    """c[M, n] = a[M, k] (f16) . (w[n, k]^T * scale[n]): the INT8 prefill
    GEMM (W8A16 on f16 MFMA), c float32 or float16; flags ST_FLAG_TILED when
    w is in the layout of st_int8_repack."""
    torch = _torch()
    m = _check_io(a, k, c, n, x_dtypes=(torch.float16,), out_dtypes=(torch.float32, torch.float16), name="a")
    nbytes = lib().st_int8_tiled_bytes(k, n) if flags & ST_FLAG_TILED else k * n
    _need(w, "w", (torch.int8,), nbytes)
    _need(scale, "scale", (torch.float32,), n)
    cd = ST_F32 if c.dtype == torch.float32 else ST_F16
    gpu.sync_stream()
    call("st_int8_gemm", gpu.handle, ptr(a), ptr(w), ptr(scale), ptr(c), cd, m, k, n, flags)


def gptq_gemm(gpu, a, qweight, scales, c, k: int, n: int, group_size: int = 128, qzeros=None, perm=None,
              flags: int = 0) -> None:
    """c[M, n] = a[M, k] (f16) . dequant(W), c float32 or float16."""
    import torch

    _check_gptq(qweight, scales, qzeros, perm, k, n, group_size, flags)
    m = _check_io(a, k, c, n, x_dtypes=(torch.float16,), out_dtypes=(torch.float32, torch.float16), name="a")
    cd = ST_F32 if c.dtype == torch.float32 else ST_F16
    gpu.sync_stream()
    call("st_gptq_i4_gemm", gpu.handle, ptr(a), ptr(qweight), ptr(scales), ptr(qzeros), ptr(perm), ptr(c), cd, m,
         k, n, group_size, flags)


def gate_up_gemm(gpu, a, gate_qw, gate_sc, up_qw, up_sc, gate_out, up_out, k: int, n: int, group_size: int = 128,
                 gate_qz=None, up_qz=None, perm=None, flags: int = 0) -> None:
    """gate_out = a . dequant(Wg) and up_out = a . dequant(Wu), [M, n] each,
    float32 or float16 (one dtype), from one pass over a (f16): the M-token
    gate and up projections of src/model.rs:803-811, each bit for bit what
    gptq_gemm gives for that weight."""
    import torch

    _check_gptq(gate_qw, gate_sc, gate_qz, perm, k, n, group_size, flags)
    _check_gptq(up_qw, up_sc, up_qz, perm, k, n, group_size, flags)
    m = _check_io(a, k, gate_out, n, x_dtypes=(torch.float16,), out_dtypes=(torch.float32, torch.float16), name="a")
    _need(up_out, "up_out", (gate_out.dtype,), m * n)
    cd = ST_F32 if gate_out.dtype == torch.float32 else ST_F16
    gpu.sync_stream()
    call("st_gptq_i4_gate_up_gemm", gpu.handle, ptr(a), ptr(gate_qw), ptr(gate_sc), ptr(gate_qz), ptr(up_qw),
         ptr(up_sc), ptr(up_qz), ptr(perm), ptr(gate_out), ptr(up_out), cd, m, k, n, group_size, flags)


def fused_silu_gptq_gemm(gpu, gate_out, up_out, down_qw, down_sc, output, k: int, n: int, group_size: int = 128,
                         qzeros=None, perm=None, flags: int = 0) -> None:
    """output[M, n] = (silu(gate_out) * up_out)[M, k] . dequant(W): the
    M-token form of fused_silu_gptq_down (src/model.rs:383-408) through the
    prefill GEMM; gate_out and up_out f16, output float32 or float16."""
    import torch

    _check_gptq(down_qw, down_sc, qzeros, perm, k, n, group_size, flags)
    m = _check_io(gate_out, k, output, n, x_dtypes=(torch.float16,), out_dtypes=(torch.float32, torch.float16),
                  name="gate_out")
    if up_out.shape != gate_out.shape:
        raise ValueError("gate_out and up_out: float16 tensors of one shape")
    _need(up_out, "up_out", (torch.float16,), m * k)
    cd = ST_F32 if output.dtype == torch.float32 else ST_F16
    gpu.sync_stream()
    call("st_gptq_i4_silu_gemm", gpu.handle, ptr(gate_out), ptr(up_out), ptr(down_qw), ptr(down_sc), ptr(qzeros),
         ptr(perm), ptr(output), cd, m, k, n, group_size, flags)


def bf16_matvec(gpu, x, w, y, k: int, n: int) -> None:
    """y[M, n] = x[M, k] . w^T, w bf16 [n, k] (Model::bf16_lm_head,
    src/model.rs:455-468 / bf16_matvec.wgsl). x f32 or f16, y f32, M <= 8."""
    import torch

    m = _check_io(x, k, y, n)
    _need(w, "w", (torch.bfloat16, torch.int16, torch.uint16), n * k)
    gpu.sync_stream()
    call("st_bf16_matvec", gpu.handle, ptr(x), _xdtype(x), ptr(w), ptr(y), m, k, n)


# ---------------------------------------------------------- weight objects
def linear(gpu, x, w, y) -> None:
    """Dispatch on the weight type: GptqWeight -> st_gptq_i4_matvec (M <= 32)
    or the prefill GEMM (M > 32: it computes on f16 activations, so f32 x is
    rounded to f16 first); Int8Weight -> st_int8_matvec (M <= 32) or
    st_int8_gemm (M > 32, likewise on f16 activations)."""
    if isinstance(w, GptqWeight):
        m = _rows(x, w.K)
        if m > 32:
            xa = x if x.dtype == _torch().float16 else x.to(_torch().float16)
            gptq_gemm(gpu, xa, w.qweight, w.scales, y, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
        else:
            gptq_matvec(gpu, "linear", x, w.qweight, w.scales, y, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
    elif isinstance(w, Int8Weight):
        m = _rows(x, w.K)
        if m > 32:
            xa = x if x.dtype == _torch().float16 else x.to(_torch().float16)
            int8_gemm(gpu, xa, w.w, w.scale, y, w.K, w.N, w.flags)
        else:
            int8_matvec(gpu, x, w.w, w.scale, y, w.K, w.N, w.flags)
    else:
        raise TypeError(type(w))
