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


def dn_parts(H=256, T=384, Z=128, I=512):
    return dict(in_qkv=w(H, T), in_z=w(H, Z), out=w(Z, H), gate=w(H, I), up=w(H, I), down=w(I, H))


def test_deltanet_construction_concatenates_qkv_and_z():
    p = dn_parts()
    layer = sta.DeltaNetLinears(**p)
    assert layer.kind == "linear_attn" and layer.qkv.N == 384 + 128 and layer.splits == (384, 128)
    assert (layer.hidden, layer.attn_dim, layer.inter) == (256, 128, 512)
    y = torch.zeros(3, layer.qkv.N)
    assert layer.z_of(y).shape == (3, 128)


@pytest.mark.parametrize("bad,shape", [("out", (256, 256)), ("out", (128, 64)), ("in_z", (128, 128)),
                                       ("down", (256, 256))])
def test_deltanet_inconsistent_shapes_are_rejected(bad, shape):
    p = dn_parts()
    p[bad] = w(*shape)
    with pytest.raises(ValueError):
        sta.DeltaNetLinears(**p)


def test_layer_kind_by_reference_names():
    """The reference's loader takes a layer as self-attention when its
    self_attn.q_proj is present (src/weights.rs:247-250), else as DeltaNet
    with linear_attn.{in_proj_qkv,in_proj_z,out_proj} (:478-483)."""
    sa, dn = parts(), dn_parts()
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    dnames = {"in_qkv": "linear_attn.in_proj_qkv", "in_z": "linear_attn.in_proj_z", "out": "linear_attn.out_proj",
              "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    linears = {f"model.layers.0.{dnames[n]}": x for n, x in dn.items()}
    linears.update({f"model.layers.1.{names[n]}": x for n, x in sa.items()})
    L0 = sta.layer_from_linears(linears, 0)
    L1 = sta.layer_from_linears(linears, 1)
    assert L0.kind == "linear_attn" and L0.o is dn["out"] and L0.down is dn["down"]
    assert L1.kind == "self_attn" and L1.o is sa["o"]
    with pytest.raises(KeyError):
        sta.DeltaNetLinears.from_linears(linears, 1)
    with pytest.raises(KeyError):
        sta.layer_from_linears(linears, 2)
    st = sta.DecoderStack.from_linears(linears, 2, w(256, 1000))
    assert [L.kind for L in st.layers] == ["linear_attn", "self_attn"] and st.vocab == 1000


def test_stack_rejects_mixed_hidden_sizes():
    with pytest.raises(ValueError):
        sta.DecoderStack([sta.DecoderLinears(**parts()), sta.DeltaNetLinears(**dn_parts(I=256))], w(256, 64))
