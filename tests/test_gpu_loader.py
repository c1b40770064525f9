"""GPTQ safetensors loader end to end on the GPU: the uploaded linears
(zeros honoured with the v1 convention, act-order sorted, tiled) and the bf16
lm_head reproduce the f64 oracle on the file's own tensors."""
import numpy as np
import pytest
import torch

from ckpt_util import write_checkpoint
import shady_thinker_amd as sta
from shady_thinker_amd import model as M
from shady_thinker_amd.loader import load_gptq_checkpoint

pytestmark = pytest.mark.gpu


def test_loaded_weights_match_oracle(gpu, orc, tmp_path):
    src = write_checkpoint(orc, str(tmp_path))
    linears, bf16 = load_gptq_checkpoint(gpu, str(tmp_path))
    q = linears["model.layers.0.self_attn.q_proj"]
    assert q.perm is None and q.tiled  # identity g_idx dropped
    assert q.qzeros is None  # symmetric v1 zeros (every stored 7 + 1 = 8) are the implicit z = 8
    x = torch.from_numpy(src["q"]["x"]).cuda()[None]
    y = torch.empty(1, 64, device="cuda")
    sta.linear(gpu, x, q, y)
    ref = orc.gptq_matvec_f64(src["q"]["x"], src["q"]["qweight"], src["q"]["scales"], 256, 64, 128,
                              qzeros=src["z7"], zero_offset=1)
    ref8 = orc.gptq_matvec_f64(src["q"]["x"], src["q"]["qweight"], src["q"]["scales"], 256, 64, 128)
    assert np.array_equal(ref, ref8)  # stored 7 + 1 = the reference's z = 8
    assert orc.rel_l2(y.cpu().numpy()[0], ref) < 1e-6
    d = linears["model.layers.0.mlp.down_proj"]
    assert d.perm is not None and d.qzeros is not None  # random zeros are kept
    dn = src["down"]
    xd = torch.from_numpy(dn["x"]).cuda()[None]
    yd = torch.empty(1, 32, device="cuda")
    sta.linear(gpu, xd, d, yd)
    refd = orc.gptq_matvec_f64(dn["x"], dn["qweight"], dn["scales"], 384, 32, 128, qzeros=dn["qzeros"],
                               g_idx=dn["g_idx"], zero_offset=1)
    assert orc.rel_l2(yd.cpu().numpy()[0], refd) < 1e-6
    w = bf16["lm_head.weight"]
    lm = src["lm"]
    xl = torch.from_numpy(lm["x"]).cuda()
    yl = torch.empty(1, 48, device="cuda")
    M.bf16_matvec(gpu, xl, w, yl, 256, 48)
    torch.cuda.synchronize()
    assert orc.rel_l2(yl.cpu().numpy()[0], orc.bf16_matvec_f64(lm["x"][0], lm["w"], 256, 48)) < 1e-6
