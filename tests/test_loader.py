"""GPTQ safetensors loader, host side (no GPU): shard discovery, names,
quantize_config.json, the zero-point convention and shape validation."""
import json
import os

import numpy as np
import pytest

from ckpt_util import write_checkpoint
from shady_thinker_amd.loader import read_gptq_checkpoint


def test_reads_linears_config_and_bf16(orc, tmp_path):
    src = write_checkpoint(orc, str(tmp_path))
    ck = read_gptq_checkpoint(str(tmp_path))
    assert [os.path.basename(s) for s in ck.shards] == ["model-00001-of-00002.safetensors",
                                                        "model-00002-of-00002.safetensors"]
    assert ck.quant.group_size == 128 and ck.quant.bits == 4
    assert ck.zeros_plus_one  # AutoGPTQ v1: stored z - 1
    assert sorted(ck.linears) == ["model.layers.0.mlp.down_proj", "model.layers.0.self_attn.q_proj"]
    q = ck.linears["model.layers.0.self_attn.q_proj"]
    assert np.array_equal(q["qweight"].view(np.uint32), src["q"]["qweight"])
    assert np.array_equal(q["scales"].view(np.uint16), src["q"]["scales"].view(np.uint16))
    assert np.array_equal(q["qzeros"].view(np.uint32), src["z7"])
    d = ck.linears["model.layers.0.mlp.down_proj"]
    assert np.array_equal(d["g_idx"], src["down"]["g_idx"])
    assert list(ck.bf16) == ["lm_head.weight"]
    assert np.array_equal(ck.bf16["lm_head.weight"], src["lm"]["w"])
    assert "model.layers.0.input_layernorm" not in ck.linears


def test_v2_format_stores_zeros_as_is(orc, tmp_path):
    write_checkpoint(orc, str(tmp_path), checkpoint_format="gptq_v2")
    assert not read_gptq_checkpoint(str(tmp_path)).zeros_plus_one


def test_rejects_group_size_mismatch_and_missing_files(orc, tmp_path):
    write_checkpoint(orc, str(tmp_path))
    cfg = os.path.join(str(tmp_path), "quantize_config.json")
    with open(cfg) as f:
        c = json.load(f)
    c["group_size"] = 64
    with open(cfg, "w") as f:
        json.dump(c, f)
    with pytest.raises(ValueError):
        read_gptq_checkpoint(str(tmp_path))
    with pytest.raises(FileNotFoundError):
        read_gptq_checkpoint(str(tmp_path / "empty"))
