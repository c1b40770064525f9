"""Seeded random shapes through every decode and prefill entry point, against
the f64 oracle: GPTQ matvec (1-32 tokens, f32 or f16 x), the fused gate/up
(1-16 tokens), the prefill GEMM (f32 or f16 C), and INT8 through linear()
(matvec up to 32 tokens, GEMM above), over group sizes 64/128/256, raw or
+1 zero points, act-order, both weight layouts and ragged N. The fixed-shape
tests pin each path; this one looks for the combination they miss.

Bars (north_star): rel-L2 1e-4 for the f32-accumulate matvec family, 2e-3
for the f16-MFMA GEMM; INT8 products are exact, so 1e-5."""
import random

import numpy as np
import pytest
import torch

import shady_thinker_amd as sta
from shady_thinker_amd import model as M

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [11, 12, 13, 14])
def test_random_shapes_match_oracle(gpu, orc, seed):
    rng = random.Random(seed)
    for it in range(10):
        gs = rng.choice([64, 128, 256])
        K = 128 * rng.randint(1, 40)
        K -= K % gs
        K = max(K, gs, 128)
        N = 8 * rng.randint(1, 900)
        Mr = rng.choice([1, 2, 3, 4, 5, 8, 12, 16, 17, 24, 32])
        zeros = rng.random() < 0.5
        plus1 = zeros and rng.random() < 0.3
        act = rng.random() < 0.3
        tiled = rng.random() < 0.8
        xf16 = rng.random() < 0.3
        case = orc.gptq_case(5000 + 100 * seed + it, K, N, gs, zeros=zeros, act_order=act, M=Mr,
                             x_dtype=np.float16 if xf16 else np.float32)
        w = sta.GptqWeight.upload(gpu, case["qweight"], case["scales"], gs, qzeros=case["qzeros"],
                                  g_idx=case["g_idx"], zeros_plus_one=plus1, tiled=tiled)
        desc = (f"seed={seed} it={it} K={K} N={N} gs={gs} M={Mr} zeros={zeros}{'+1' if plus1 else ''} "
                f"act={act} tiled={tiled} x={'f16' if xf16 else 'f32'}")
        print(desc, flush=True)
        ref = orc.gptq_matvec_f64(case["x"], case["qweight"], case["scales"], K, N, gs, qzeros=case["qzeros"],
                                  g_idx=case["g_idx"], zero_offset=int(plus1))
        x = torch.from_numpy(case["x"]).cuda()
        y = torch.full((Mr, N), float("nan"), device="cuda")
        M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y, K, N, gs, w.qzeros, w.perm, w.flags)
        torch.cuda.synchronize()
        assert orc.rel_l2(y.cpu().numpy(), ref) < 1e-4, desc
        if N % 16 == 0 or not tiled:  # gate = up = w: silu(y) * y
            g = torch.full((Mr, N), float("nan"), device="cuda")
            M.fused_gate_up_silu(gpu, x, w.qweight, w.scales, w.qweight, w.scales, g, K, N, gs, w.qzeros, w.qzeros,
                                 w.perm, w.flags)
            torch.cuda.synchronize()
            assert orc.rel_l2(g.cpu().numpy(), ref / (1.0 + np.exp(-ref)) * ref) < 1e-4, desc
        Mg = rng.choice([33, 64, 100, 129, 257])
        a = torch.randn(Mg, K, generator=torch.Generator().manual_seed(seed * 100 + it)).half()
        cg = torch.full((Mg, N), float("nan"), device="cuda", dtype=rng.choice([torch.float32, torch.float16]))
        M.gptq_gemm(gpu, a.cuda(), w.qweight, w.scales, cg, K, N, gs, w.qzeros, w.perm, w.flags)
        torch.cuda.synchronize()
        rg = orc.gptq_matvec_f64(a.numpy(), case["qweight"], case["scales"], K, N, gs, qzeros=case["qzeros"],
                                 g_idx=case["g_idx"], zero_offset=int(plus1))
        assert orc.rel_l2(cg.float().cpu().numpy(), rg) < 2e-3, desc + f" Mg={Mg} {cg.dtype}"
        K8, N8 = 128 * rng.randint(1, 30), 4 * rng.randint(1, 2000)
        M8 = rng.choice([1, 2, 5, 8, 16, 32, 48, 130])
        c8 = orc.int8_case(6000 + 100 * seed + it, K8, N8, M=M8)
        w8 = sta.Int8Weight.upload(gpu, c8["w"], c8["scale"], tiled=rng.random() < 0.7)
        y8 = torch.full((M8, N8), float("nan"), device="cuda")
        M.linear(gpu, torch.from_numpy(c8["x"]).cuda(), w8, y8)
        torch.cuda.synchronize()
        r8 = orc.int8_matvec_f64(c8["x"], c8["w"], c8["scale"], K8, N8)
        assert orc.rel_l2(y8.cpu().numpy(), r8) < 1e-5, f"int8 K={K8} N={N8} M={M8} flags={w8.flags}"
