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

from ._lib import ST_F16, ST_F32, call
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
    if t.numel() % k:
        raise ValueError(f"input of {t.numel()} elements is not [M, {k}]")
    return t.numel() // k


def gptq_matvec(gpu, name: str, input, qweight, scales, output, k: int, n: int, group_size: int = 128,
                qzeros=None, perm=None, flags: int = 0) -> None:
    """output[M, n] = input[M, k] . dequant(W)  (src/model.rs:357-381)."""
    m = _rows(input, k)
    gpu.sync_stream()
    call("st_gptq_i4_matvec", gpu.handle, ptr(input), _xdtype(input), ptr(qweight), ptr(scales), ptr(qzeros),
         ptr(perm), ptr(output), m, k, n, group_size, flags)


def fused_silu_gptq_down(gpu, gate_out, up_out, down_qw, down_sc, output, k: int, n: int, group_size: int = 128,
                         qzeros=None, perm=None, flags: int = 0) -> None:
    """output = (silu(gate_out) * up_out) . dequant(W_down)  (src/model.rs:383-408)."""
    m = _rows(gate_out, k)
    gpu.sync_stream()
    call("st_gptq_i4_silu_matvec", gpu.handle, ptr(gate_out), ptr(up_out), ptr(down_qw), ptr(down_sc),
         ptr(qzeros), ptr(perm), ptr(output), m, k, n, group_size, flags)


def fused_gate_up_silu(gpu, input, gate_qw, gate_sc, up_qw, up_sc, output, k: int, n: int, group_size: int = 128,
                       gate_qz=None, up_qz=None, perm=None, flags: int = 0) -> None:
    """output = silu(input . Wg) * (input . Wu)  (fused_gate_up_silu_4t.wgsl)."""
    m = _rows(input, k)
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
    gpu.sync_stream()
    call("st_gptq_i4_dequant", gpu.handle, ptr(qweight), ptr(scales), ptr(qzeros), ptr(g_idx), ptr(out), od, k, n,
         group_size, flags)


def int8_matvec(gpu, x, w, scale, y, k: int, n: int, flags: int = 0) -> None:
    """y[M, n] = x[M, k] . (w[n, k]^T * scale[n]) (INT8 per-channel); flags
    ST_FLAG_TILED when w is in the layout of st_int8_repack."""
    m = _rows(x, k)
    gpu.sync_stream()
    call("st_int8_matvec", gpu.handle, ptr(x), _xdtype(x), ptr(w), ptr(scale), ptr(y), m, k, n, flags)


def gptq_gemm(gpu, a, qweight, scales, c, k: int, n: int, group_size: int = 128, qzeros=None, perm=None,
              flags: int = 0) -> None:
    """c[M, n] = a[M, k] (f16) . dequant(W), c float32 or float16."""
    import torch

    m = _rows(a, k)
    cd = {torch.float32: ST_F32, torch.float16: ST_F16}.get(c.dtype)
    if cd is None:
        raise TypeError(f"gemm output dtype {c.dtype}")
    gpu.sync_stream()
    call("st_gptq_i4_gemm", gpu.handle, ptr(a), ptr(qweight), ptr(scales), ptr(qzeros), ptr(perm), ptr(c), cd, m,
         k, n, group_size, flags)


def fused_silu_gptq_gemm(gpu, gate_out, up_out, down_qw, down_sc, output, k: int, n: int, group_size: int = 128,
                         qzeros=None, perm=None, flags: int = 0) -> None:
    """output[M, n] = (silu(gate_out) * up_out)[M, k] . dequant(W): the
    M-token form of fused_silu_gptq_down (src/model.rs:383-408) through the
    prefill GEMM; gate_out and up_out f16, output float32 or float16."""
    import torch

    m = _rows(gate_out, k)
    if up_out.shape != gate_out.shape or gate_out.dtype != torch.float16 or up_out.dtype != torch.float16:
        raise TypeError("gate_out and up_out: float16 tensors of one shape")
    cd = {torch.float32: ST_F32, torch.float16: ST_F16}.get(output.dtype)
    if cd is None:
        raise TypeError(f"gemm output dtype {output.dtype}")
    gpu.sync_stream()
    call("st_gptq_i4_silu_gemm", gpu.handle, ptr(gate_out), ptr(up_out), ptr(down_qw), ptr(down_sc), ptr(qzeros),
         ptr(perm), ptr(output), cd, m, k, n, group_size, flags)


def bf16_matvec(gpu, x, w, y, k: int, n: int) -> None:
    """y[M, n] = x[M, k] . w^T, w bf16 [n, k] (Model::bf16_lm_head,
    src/model.rs:455-468 / bf16_matvec.wgsl). x f32 or f16, y f32, M <= 8."""
    import torch

    m = _rows(x, k)
    if w.dtype not in (torch.bfloat16, torch.int16, torch.uint16):
        raise TypeError(f"bf16 weight dtype {w.dtype}")
    gpu.sync_stream()
    call("st_bf16_matvec", gpu.handle, ptr(x), _xdtype(x), ptr(w), ptr(y), m, k, n)


# ---------------------------------------------------------- weight objects
def linear(gpu, x, w, y) -> None:
    """Dispatch on the weight type: GptqWeight -> st_gptq_i4_matvec (M <= 32)
    or the prefill GEMM (M > 32, f16 x); Int8Weight -> st_int8_matvec."""
    if isinstance(w, GptqWeight):
        m = _rows(x, w.K)
        if m > 32:
            gptq_gemm(gpu, x, w.qweight, w.scales, y, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
        else:
            gptq_matvec(gpu, "linear", x, w.qweight, w.scales, y, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
    elif isinstance(w, Int8Weight):
        int8_matvec(gpu, x, w.w, w.scale, y, w.K, w.N, w.flags)
    else:
        raise TypeError(type(w))
