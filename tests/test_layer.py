"""CPU checks of DecoderLinears' host logic: shape validation, the q|k|v
concatenation and the lookup by the reference loader's tensor names (no
kernel runs here)."""
import pytest
import torch

import shady_thinker_amd as sta
from shady_thinker_amd._lib import ST_FLAG_TILED


def w(k, n, gs=128):
    return sta.GptqWeight(torch.zeros((n + 15) // 16 * 16 * k // 8, dtype=torch.int32),
                          torch.zeros(k // gs, n, dtype=torch.float16), None, None, k, n, gs, ST_FLAG_TILED)


def parts(H=256, Q=256, KV=128, I=512):
    return dict(q=w(H, Q), k=w(H, KV), v=w(H, KV), o=w(Q, H), gate=w(H, I), up=w(H, I), down=w(I, H))


def test_construction_concatenates_qkv():
    p = parts()
    layer = sta.DecoderLinears(**p)
    assert layer.qkv.N == 256 + 2 * 128 and layer.splits == (256, 128, 128)
    assert (layer.hidden, layer.attn_dim, layer.inter) == (256, 256, 512)
    assert layer.qkv.qweight.numel() == sum(p[n].qweight.numel() for n in "qkv")


@pytest.mark.parametrize("bad", ["down", "o", "up"])
def test_inconsistent_shapes_are_rejected(bad):
    p = parts()
    p[bad] = w(256, 64)
    with pytest.raises(ValueError):
        sta.DecoderLinears(**p)


def test_gate_and_up_must_share_act_order():
    p = parts()
    p["gate"].perm = torch.arange(256, dtype=torch.int32)
    with pytest.raises(ValueError):
        sta.DecoderLinears(**p)


def test_from_linears_by_reference_names():
    p = parts()
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    linears = {f"model.language_model.layers.7.{names[n]}": x for n, x in p.items()}
    layer = sta.DecoderLinears.from_linears(linears, 7, layer_prefix="model.language_model.layers")
    assert layer.down is p["down"] and layer.o is p["o"]
    with pytest.raises(KeyError):
        sta.DecoderLinears.from_linears(linears, 6, layer_prefix="model.language_model.layers")


def test_decode_token_limit():
    layer = sta.DecoderLinears(**parts())
    with pytest.raises(ValueError):
        layer.decode(None, torch.zeros(33, 256), torch.zeros(33, 256), None, None, None, None)
