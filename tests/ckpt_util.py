"""Synthetic GPTQ checkpoints for the loader tests (written with the
safetensors library, AutoGPTQ naming and quantize_config.json)."""
import json
import os

import numpy as np


def write_checkpoint(orc, d, checkpoint_format="gptq"):
    """Two shards: layer 0 q_proj (symmetric, identity g_idx, v1 zeros = 7)
    and down_proj (act-order g_idx, random zeros), plus a bf16 lm_head and a
    norm weight that the loader must ignore. Returns the source arrays."""
    import torch
    from safetensors.torch import save_file

    gs = 128
    q = orc.gptq_case(40, 256, 64, gs)
    dn = orc.gptq_case(41, 384, 32, gs, zeros=True, act_order=True)
    G = 256 // gs
    z7 = np.full((G, 64 // 8), 0x77777777, np.uint32)
    lm = orc.bf16_case(42, 256, 48)
    as_t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).view(dt))
    shard0 = {
        "model.layers.0.self_attn.q_proj.qweight": as_t(q["qweight"], np.int32),
        "model.layers.0.self_attn.q_proj.scales": as_t(q["scales"], np.float16),
        "model.layers.0.self_attn.q_proj.qzeros": as_t(z7, np.int32),
        "model.layers.0.self_attn.q_proj.g_idx": torch.from_numpy((np.arange(256) // gs).astype(np.int32)),
        "model.layers.0.input_layernorm.weight": torch.ones(256),
    }
    shard1 = {
        "model.layers.0.mlp.down_proj.qweight": as_t(dn["qweight"], np.int32),
        "model.layers.0.mlp.down_proj.scales": as_t(dn["scales"], np.float16),
        "model.layers.0.mlp.down_proj.qzeros": as_t(dn["qzeros"], np.int32),
        "model.layers.0.mlp.down_proj.g_idx": torch.from_numpy(dn["g_idx"].astype(np.int32)),
        "lm_head.weight": as_t(lm["w"], np.int16).view(torch.bfloat16),
    }
    os.makedirs(d, exist_ok=True)
    save_file(shard0, os.path.join(d, "model-00001-of-00002.safetensors"))
    save_file(shard1, os.path.join(d, "model-00002-of-00002.safetensors"))
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": {}}, f)
    with open(os.path.join(d, "quantize_config.json"), "w") as f:
        json.dump({"bits": 4, "group_size": gs, "sym": False, "desc_act": True,
                   "checkpoint_format": checkpoint_format}, f)
    return {"q": q, "z7": z7, "down": dn, "lm": lm}
