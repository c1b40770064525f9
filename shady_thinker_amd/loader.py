"""GPTQ safetensors checkpoints -> device weights for this backend.

Mirrors the reference loader for the quantized linears (`load_weights`,
src/weights.rs:315-547): every `*.safetensors` shard in the model directory
(not the `.index.` file), in sorted order, tensors taken by name
(`{prefix}.qweight`, `{prefix}.scales`). Unlike the reference, which skips
`.qzeros` and `.g_idx` (src/weights.rs:372-374) and so assumes symmetric,
non-act-order files, this loader honours both:

* qzeros: AutoGPTQ "gptq" (v1) files store z - 1, "gptq_v2" files store z
  (`checkpoint_format` in quantize_config.json; v1 when absent). A symmetric v1
  file stores 7 everywhere, i.e. z = 8, the reference's constant.
* g_idx: an identity map (g_idx[k] = k // group_size) is dropped; any other
  sorts K by group at upload (st_gptq_i4_act_order).

Files are read with the safetensors library (no pickle). Only GPTQ linears
and bf16 2-D weights named like the lm_head / embeddings are returned; norms,
attention and the rest are outside this path.
"""
from __future__ import annotations

import glob
import json
import os
from dataclasses import dataclass, field

import numpy as np

from .weights import GptqWeight, QuantConfig, check_gptq_tensors

_GPTQ_PARTS = ("qweight", "scales", "qzeros", "g_idx")


@dataclass
class GptqCheckpoint:
    """Host-side contents of a checkpoint's quantized linears."""

    quant: QuantConfig
    zeros_plus_one: bool
    linears: dict = field(default_factory=dict)  # prefix -> {"qweight", "scales", "qzeros", "g_idx"} numpy
    bf16: dict = field(default_factory=dict)  # name -> uint16 numpy [N, K] (lm_head / embed_tokens)
    shards: list = field(default_factory=list)


def _shards(model_dir: str) -> list:
    files = sorted(p for p in glob.glob(os.path.join(model_dir, "*.safetensors")) if ".index." not in p)
    if not files:
        raise FileNotFoundError(f"no *.safetensors shards in {model_dir}")
    return files


def _quant_config(model_dir: str) -> tuple[QuantConfig, bool]:
    path = os.path.join(model_dir, "quantize_config.json")
    raw = {}
    if os.path.exists(path):
        with open(path) as f:
            raw = json.load(f)
    qc = QuantConfig.from_dict(raw)
    if qc.bits != 4:
        raise ValueError(f"quantize_config.json: bits={qc.bits}, only 4-bit GPTQ is supported")
    v2 = str(raw.get("checkpoint_format", "gptq")).lower() == "gptq_v2"
    return qc, not v2


def read_gptq_checkpoint(model_dir: str) -> GptqCheckpoint:
    """Parse the shards and quantize_config.json on the host (no GPU)."""
    from safetensors import safe_open

    qc, zp1 = _quant_config(model_dir)
    ck = GptqCheckpoint(quant=qc, zeros_plus_one=zp1, shards=_shards(model_dir))
    for path in ck.shards:
        with safe_open(path, framework="pt") as f:
            for name in f.keys():
                stem, _, part = name.rpartition(".")
                if part in _GPTQ_PARTS:
                    t = f.get_tensor(name)
                    if t.dtype == _bf16():
                        raise ValueError(f"{name}: bfloat16; GPTQ {part} must be float16 (scales) or integer")
                    ck.linears.setdefault(stem, {})[part] = t.numpy()
                elif part == "weight" and ("lm_head" in stem or "embed_tokens" in stem):
                    t = f.get_tensor(name)
                    if t.dtype == _bf16() and t.dim() == 2:
                        import torch

                        ck.bf16[name] = t.view(torch.int16).numpy().view(np.uint16)
    for stem, parts in list(ck.linears.items()):
        if "qweight" not in parts or "scales" not in parts:
            raise ValueError(f"{stem}: GPTQ tensors incomplete ({sorted(parts)}), need qweight and scales")
        qw, sc = parts["qweight"], parts["scales"]
        if qw.ndim != 2 or sc.ndim != 2 or sc.shape[1] != qw.shape[1]:
            raise ValueError(f"{stem}: qweight {qw.shape} / scales {sc.shape} do not match")
        K = qw.shape[0] * 8
        if K % sc.shape[0] or K // sc.shape[0] != qc.group_size:
            raise ValueError(f"{stem}: K={K} with {sc.shape[0]} groups, quantize_config group_size={qc.group_size}")
        try:
            check_gptq_tensors(qw, sc, qc.group_size, parts.get("qzeros"), parts.get("g_idx"))
        except ValueError as e:
            raise ValueError(f"{stem}: {e}") from None
    return ck


def _bf16():
    import torch

    return torch.bfloat16


def load_gptq_checkpoint(gpu, model_dir: str, tiled: bool = True) -> tuple[dict, dict]:
    """Upload every GPTQ linear (`{prefix: GptqWeight}`) and the bf16
    lm_head / embedding weights (`{name: device int16 tensor [N, K]}`)."""
    ck = read_gptq_checkpoint(model_dir)
    linears = {}
    for stem, p in ck.linears.items():
        qz = p.get("qzeros")
        linears[stem] = GptqWeight.upload(gpu, p["qweight"], p["scales"], ck.quant.group_size, qzeros=qz,
                                          g_idx=p.get("g_idx"), zeros_plus_one=ck.zeros_plus_one and qz is not None,
                                          tiled=tiled)
    torch = gpu.torch
    bf16 = {name: torch.from_numpy(w.view(np.int16)).to(gpu.device) for name, w in ck.bf16.items()}
    return linears, bf16
