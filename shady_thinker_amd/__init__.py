"""shady_thinker_amd: MI355X (gfx950) quantized-linear backend for shady-thinker.

The compute path is libshady_hip.so (hand-written HIP, C ABI in
include/shady_hip.h). This package is the host-side mirror of the
reference's linear-layer interface (src/gpu.rs GpuContext, src/model.rs
gptq_matvec / fused_silu_gptq_down, src/weights.rs QuantConfig).
"""
from ._lib import ST_FLAG_TILED, ST_FLAG_ZEROS_PLUS_ONE, ShadyHipError, header_symbols, lib  # noqa: F401
from .gpu import GpuContext  # noqa: F401
from .model import (  # noqa: F401
    bf16_matvec,
    fused_gate_up_silu,
    fused_silu_gptq_down,
    fused_silu_gptq_gemm,
    gptq_dequant,
    gptq_gemm,
    gptq_matvec,
    int8_matvec,
    linear,
)
from .layer import DecoderLinears, DecoderStack, DeltaNetLinears, StackBuffers, StackGraph, layer_from_linears  # noqa: F401
from .loader import load_gptq_checkpoint, read_gptq_checkpoint  # noqa: F401
from .weights import GptqWeight, Int8Weight, QuantConfig  # noqa: F401
