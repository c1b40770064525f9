"""GPU parity of the decode kernels (st_gptq_i4_matvec / _silu_matvec /
_gate_up_silu, st_int8_matvec) against the CPU oracle, through the C ABI.

Bars (stated in BASELINE.json north_star): matvec outputs within rel-L2
1e-4 of the float64 oracle and of the reference's WGSL-order f32 path;
dequantized weights bit-exact (one-hot inputs return dequantized rows
exactly).
"""
import os

import numpy as np
import pytest
import torch

import shady_thinker_amd as sta
from shady_thinker_amd import model as M

pytestmark = pytest.mark.gpu

TOL = 1e-4  # rel-L2, f32-accumulate matvec (north_star)
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def up(gpu, case, zeros_plus_one=False, tiled=True):
    return sta.GptqWeight.upload(gpu, case["qweight"], case["scales"], case["gs"], qzeros=case["qzeros"],
                                 g_idx=case["g_idx"], zeros_plus_one=zeros_plus_one, tiled=tiled)


def run_matvec(gpu, w, x_np, dtype=torch.float32):
    x = torch.from_numpy(np.ascontiguousarray(x_np)).to(gpu.device)
    if dtype == torch.float16:
        x = x.half()
    m = x.numel() // w.K
    y = torch.empty(m, w.N, dtype=torch.float32, device=gpu.device)
    M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y, w.K, w.N, w.group_size, w.qzeros, w.perm, w.flags)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_cfg1_matches_oracle_and_wgsl(gpu, orc):
    K = N = 2048
    c = orc.gptq_case(0, K, N, 128)
    w = up(gpu, c)
    y = run_matvec(gpu, w, c["x"])[0]
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, 128)
    wg = orc.gptq_matvec_wgsl(c["x"], c["qweight"], c["scales"], K, N, 128, 1, 1)
    e64, ewg = orc.rel_l2(y, ref), orc.rel_l2(y, wg)
    print(f"cfg1 rel-L2 vs f64 {e64:.3e}, vs WGSL-4t {ewg:.3e}")
    assert e64 < TOL and ewg < TOL
    assert e64 < 1e-6  # the integer-limb scheme is far tighter than the bar


def test_one_hot_returns_dequant_rows_exactly(gpu, orc):
    K, N, gs = 1024, 264, 128
    c = orc.gptq_case(1, K, N, gs, zeros=True)
    w = up(gpu, c)
    W = orc.gptq_dequant_f32(c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"])
    ks = [0, 1, 7, 8, 127, 128, 500, 1023]
    x = np.zeros((len(ks), K), np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    y = run_matvec(gpu, w, x)
    assert np.array_equal(y, W[ks]), "dequantized rows must be bit-exact"
    # a power-of-two scaled one-hot too (the per-group exponent path)
    y2 = run_matvec(gpu, w, x * np.float32(2.0 ** -30))
    assert np.array_equal(y2, W[ks] * np.float32(2.0 ** -30))


def test_integer_exact_case_bit_equal(gpu, orc):
    K, N, gs = 2048, 512, 128
    c = orc.gptq_case(2, K, N, gs)
    c["scales"] = np.ones_like(c["scales"])
    x = np.round(c["x"] * 4).astype(np.float32)
    w = up(gpu, c)
    y = run_matvec(gpu, w, x)[0]
    ref = orc.gptq_matvec_f64(x, c["qweight"], c["scales"], K, N, gs)
    assert np.array_equal(y.astype(np.float64), ref)


@pytest.mark.parametrize("K,N,gs,Mr", [
    (128, 8, 128, 1), (256, 64, 64, 1), (512, 264, 128, 1), (4096, 4096, 128, 1), (11008, 4096, 128, 1),
    (2560, 1032, 256, 1), (4096, 2048, 128, 2), (2048, 520, 128, 3), (2048, 1024, 64, 5), (4096, 512, 128, 8),
    (2560, 1024, 128, 16), (1024, 256, 128, 32),
])
def test_shapes_vs_f64(gpu, orc, K, N, gs, Mr):
    c = orc.gptq_case(K + N + Mr, K, N, gs, M=Mr)
    w = up(gpu, c)
    y = run_matvec(gpu, w, c["x"])
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs)
    assert y.shape == (Mr, N)
    e = orc.rel_l2(y, ref)
    print(f"K={K} N={N} gs={gs} M={Mr}: rel-L2 {e:.3e}")
    assert e < TOL
    for m in range(Mr):  # every row individually too
        assert orc.rel_l2(y[m], ref[m]) < TOL


def test_f16_activations(gpu, orc):
    K, N = 4096, 4096
    c = orc.gptq_case(31, K, N, 128, x_dtype=np.float16)
    w = up(gpu, c)
    y = run_matvec(gpu, w, c["x"], dtype=torch.float16)[0]
    ref = orc.gptq_matvec_f64(c["x"].astype(np.float64), c["qweight"], c["scales"], K, N, 128)
    assert orc.rel_l2(y, ref) < TOL


@pytest.mark.parametrize("plus_one", [False, True])
def test_zero_points(gpu, orc, plus_one):
    K, N, gs = 4096, 1024, 128
    c = orc.gptq_case(41, K, N, gs, zeros=True, M=2)
    w = up(gpu, c, zeros_plus_one=plus_one)
    y = run_matvec(gpu, w, c["x"])
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"],
                              zero_offset=int(plus_one))
    assert orc.rel_l2(y, ref) < TOL


@pytest.mark.parametrize("plus_one", [False, True])
def test_symmetric_zeros_not_uploaded(gpu, orc, plus_one):
    """qzeros that are all 8 (all 7 with the v1 +1 convention) are dropped at
    upload: the kernels' implicit z = 8 gives the same bits as the explicit
    table (matvec, gate/up and the GEMM), and the oracle's result."""
    K, N, gs = 2048, 1024, 128
    c = orc.gptq_case(44, K, N, gs, M=3)
    z = np.full((K // gs, N // 8), 0x77777777 if plus_one else 0x88888888, np.uint32)
    kw = dict(zeros_plus_one=plus_one)
    w_drop = sta.GptqWeight.upload(gpu, c["qweight"], c["scales"], gs, qzeros=z, **kw)
    w_keep = sta.GptqWeight.upload(gpu, c["qweight"], c["scales"], gs, qzeros=z, drop_symmetric_zeros=False, **kw)
    assert w_drop.qzeros is None and w_keep.qzeros is not None
    y_drop, y_keep = run_matvec(gpu, w_drop, c["x"]), run_matvec(gpu, w_keep, c["x"])
    assert np.array_equal(y_drop, y_keep)
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=z, zero_offset=int(plus_one))
    assert orc.rel_l2(y_drop, ref) < TOL
    x = torch.from_numpy(c["x"]).cuda()
    outs = []
    for w in (w_drop, w_keep):
        g = torch.empty(3, N, device="cuda")
        M.fused_gate_up_silu(gpu, x, w.qweight, w.scales, w.qweight, w.scales, g, K, N, gs, w.qzeros, w.qzeros,
                             None, w.flags)
        a = torch.randn(48, K, generator=torch.Generator().manual_seed(1)).half().cuda()
        cg = torch.empty(48, N, device="cuda")
        M.gptq_gemm(gpu, a, w.qweight, w.scales, cg, K, N, gs, w.qzeros, None, w.flags)
        torch.cuda.synchronize()
        outs.append((g.cpu(), cg.cpu()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_act_order(gpu, orc):
    K, N, gs = 4096, 2048, 128
    c = orc.gptq_case(51, K, N, gs, zeros=True, act_order=True)
    w = up(gpu, c)
    assert w.perm is not None
    y = run_matvec(gpu, w, c["x"])[0]
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
    assert orc.rel_l2(y, ref) < TOL
    # identity g_idx is detected and needs no permutation
    c2 = dict(c, g_idx=(np.arange(K) // gs).astype(np.int32))
    assert up(gpu, c2).perm is None


def test_act_order_sorted_weights_dequantize_identically(gpu, orc):
    K, N, gs = 1024, 128, 128
    c = orc.gptq_case(52, K, N, gs, act_order=True)
    w = up(gpu, c, tiled=False)
    perm = w.perm.cpu().numpy()
    qs = w.qweight.cpu().numpy().view(np.uint32)
    W = orc.gptq_dequant_f32(c["qweight"], c["scales"], K, N, gs, g_idx=c["g_idx"])
    Ws = orc.gptq_dequant_f32(qs, c["scales"], K, N, gs)  # sorted: group = k // gs
    assert np.array_equal(Ws, W[perm])
    assert np.array_equal(np.sort(perm), np.arange(K))
    assert np.all(np.diff(c["g_idx"][perm]) >= 0)


def test_act_order_rejects_unequal_groups(gpu, orc):
    K, N, gs = 256, 64, 128
    c = orc.gptq_case(53, K, N, gs)
    bad = np.zeros(K, np.int32)  # all rows in group 0
    with pytest.raises(sta.ShadyHipError) as ei:
        sta.GptqWeight.upload(gpu, c["qweight"], c["scales"], gs, g_idx=bad)
    assert ei.value.code == 2


def test_fused_silu_down(gpu, orc):
    K, N, gs = 11008, 4096, 128
    c = orc.gptq_case(61, K, N, gs)
    a = orc.normal_f32(610, K) * 2
    b = orc.normal_f32(611, K)
    w = up(gpu, c)
    da = torch.from_numpy(a).cuda()
    db = torch.from_numpy(b).cuda()
    y = torch.empty(1, N, device="cuda")
    M.fused_silu_gptq_down(gpu, da, db, w.qweight, w.scales, y, K, N, gs, flags=w.flags)
    torch.cuda.synchronize()
    y = y.cpu().numpy()[0]
    ref = orc.gptq_matvec_f64(orc.silu_mul_f64(a, b), c["qweight"], c["scales"], K, N, gs)
    wg = orc.fused_silu_gptq_wgsl(a, b, c["qweight"], c["scales"], K, N, gs, 1, 1)
    assert orc.rel_l2(y, ref) < TOL and orc.rel_l2(y, wg) < TOL
    # a = 0 -> silu = 0 -> y = 0 exactly
    y0 = torch.full((1, N), 5.0, device="cuda")
    M.fused_silu_gptq_down(gpu, torch.zeros(K, device="cuda"), db, w.qweight, w.scales, y0, K, N, gs, flags=w.flags)
    torch.cuda.synchronize()
    assert torch.count_nonzero(y0).item() == 0


@pytest.mark.parametrize("Mr", [1, 4, 16])
def test_gate_up_silu(gpu, orc, Mr):
    K, N, gs = 4096, 11008, 128
    cg = orc.gptq_case(71, K, N, gs, M=Mr)
    cu = orc.gptq_case(72, K, N, gs)
    wg_, wu_ = up(gpu, cg), up(gpu, cu)
    x = torch.from_numpy(cg["x"]).cuda()
    y = torch.empty(Mr, N, device="cuda")
    M.fused_gate_up_silu(gpu, x, wg_.qweight, wg_.scales, wu_.qweight, wu_.scales, y, K, N, gs, flags=wg_.flags)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    g = orc.gptq_matvec_f64(cg["x"], cg["qweight"], cg["scales"], K, N, gs)
    u = orc.gptq_matvec_f64(cg["x"], cu["qweight"], cu["scales"], K, N, gs)
    ref = orc.silu_gate_f64(g, u)
    assert orc.rel_l2(y, ref) < TOL
    if Mr == 1:
        wgsl = orc.gate_up_silu_wgsl(cg["x"], cg["qweight"], cg["scales"], cu["qweight"], cu["scales"], K, N, gs, 1, 1)
        assert orc.rel_l2(y[0], wgsl) < TOL


@pytest.mark.parametrize("Mr", [1, 8, 32])
def test_int8_cfg3(gpu, orc, Mr):
    K, N = 5120, 13824
    c = orc.int8_case(81, K, N, M=Mr)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
    x = torch.from_numpy(c["x"]).cuda()
    y = torch.empty(Mr, N, device="cuda")
    M.int8_matvec(gpu, x, w.w, w.scale, y, K, N, w.flags)
    torch.cuda.synchronize()
    ref = orc.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)
    e = orc.rel_l2(y.cpu().numpy(), ref)
    print(f"int8 M={Mr} rel-L2 {e:.3e}")
    assert e < TOL


def test_int8_f32_small_ragged(gpu, orc):
    K, N = 384, 36
    c = orc.int8_case(82, K, N, M=3, x_dtype=np.float32)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
    y = torch.empty(3, N, device="cuda")
    M.int8_matvec(gpu, torch.from_numpy(c["x"]).cuda(), w.w, w.scale, y, K, N, w.flags)
    torch.cuda.synchronize()
    assert orc.rel_l2(y.cpu().numpy(), orc.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)) < TOL


def test_golden_fixtures(gpu, orc):
    for f in sorted(os.listdir(GOLDEN)):
        if not f.endswith(".npz"):
            continue
        d = np.load(os.path.join(GOLDEN, f))
        kind, K, N = str(d["kind"]), int(d["K"]), int(d["N"])
        if kind == "int8":
            w = sta.Int8Weight.upload(gpu, d["w"], d["scale"])
            x = torch.from_numpy(d["x"]).cuda()
            y = torch.empty(d["y"].shape, device="cuda")
            M.int8_matvec(gpu, x, w.w, w.scale, y, K, N, w.flags)
        else:
            gs = int(d["gs"])
            w = sta.GptqWeight.upload(gpu, d["qweight"], d["scales"], gs,
                                      qzeros=d["qzeros"] if d["qzeros"].size else None,
                                      g_idx=d["g_idx"] if d["g_idx"].size else None)
            y = torch.empty(d["y"].shape, device="cuda")
            if kind == "silu":
                M.fused_silu_gptq_down(gpu, torch.from_numpy(d["a"]).cuda(), torch.from_numpy(d["b"]).cuda(),
                                       w.qweight, w.scales, y, K, N, gs, w.qzeros, w.perm, w.flags)
            else:
                M.gptq_matvec(gpu, "golden", torch.from_numpy(d["x"]).cuda(), w.qweight, w.scales, y, K, N, gs,
                              w.qzeros, w.perm, w.flags)
        torch.cuda.synchronize()
        e = orc.rel_l2(y.cpu().numpy(), d["y"])
        assert e < TOL, (f, e)


def test_deterministic_and_split_consistent(gpu, orc, tune):
    K, N = 11008, 4096
    c = orc.gptq_case(91, K, N, 128)
    w = up(gpu, c)
    y1 = run_matvec(gpu, w, c["x"])
    y2 = run_matvec(gpu, w, c["x"])
    assert np.array_equal(y1, y2)


def test_nonfinite_input_poisons_output(gpu, orc):
    K, N = 512, 64
    c = orc.gptq_case(92, K, N, 128)
    w = up(gpu, c)
    x = c["x"].copy()
    x[300] = np.nan
    y = run_matvec(gpu, w, x)[0]
    assert np.all(np.isnan(y))


def test_bad_shapes_raise(gpu, orc):
    c = orc.gptq_case(93, 256, 64, 128)
    w = up(gpu, c)
    x = torch.zeros(256, device="cuda")
    y = torch.empty(64, device="cuda")
    gpu.sync_stream()
    # an unsupported group size, at the C ABI (the Python helper refuses it
    # earlier: its scales would be too short)
    rc = sta._lib.lib().st_gptq_i4_matvec(gpu.handle, x.data_ptr(), 0, w.qweight.data_ptr(), w.scales.data_ptr(),
                                          None, None, y.data_ptr(), 1, 256, 64, 32, w.flags)
    assert rc == 2  # ST_ERR_SHAPE
    with pytest.raises(ValueError):
        M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y, 256, 64, 32, flags=w.flags)
    with pytest.raises(sta.ShadyHipError) as ei:
        M.gptq_matvec(gpu, "t", torch.zeros(40 * 256, device="cuda"), w.qweight, w.scales,
                      torch.empty(40 * 64, device="cuda"), 256, 64, 128, flags=w.flags)  # M=40
    assert ei.value.code == 2


def test_dequant_kernel_bit_exact(gpu, orc):
    K, N, gs = 1024, 192, 128
    for zeros, act in [(False, False), (True, False), (True, True)]:
        c = orc.gptq_case(94, K, N, gs, zeros=zeros, act_order=act)
        qw = gpu.upload_array(c["qweight"].view(np.int32), torch.int32)
        sc = gpu.upload_array(c["scales"], torch.float16)
        qz = None if c["qzeros"] is None else gpu.upload_array(c["qzeros"].view(np.int32), torch.int32)
        gi = None if c["g_idx"] is None else gpu.upload_array(c["g_idx"], torch.int32)
        out = torch.empty(K, N, device="cuda")
        M.gptq_dequant(gpu, qw, sc, out, K, N, gs, qz, gi)
        ob = torch.empty(K, N, device="cuda", dtype=torch.bfloat16)
        M.gptq_dequant(gpu, qw, sc, ob, K, N, gs, qz, gi)
        torch.cuda.synchronize()
        ref = orc.gptq_dequant_f32(c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))
        if not zeros:
            refb = orc.gptq_dequant_bf16(c["qweight"], c["scales"], K, N, gs)
            assert np.array_equal(ob.cpu().view(torch.int16).numpy().view(np.uint16), refb)


@pytest.mark.parametrize("K,N,gs,Mr,zeros", [(4096, 4096, 128, 1, False), (2048, 264, 64, 3, True),
                                             (2560, 1032, 256, 5, False), (1024, 136, 128, 16, True)])
def test_reference_and_tiled_layouts_agree(gpu, orc, K, N, gs, Mr, zeros):
    """Both layouts give the same group results; only the split of K among
    waves (hence the f32 order of the cross-wave sum) may differ."""
    c = orc.gptq_case(K + Mr, K, N, gs, zeros=zeros, M=Mr)
    yr = run_matvec(gpu, up(gpu, c, tiled=False), c["x"])
    yt = run_matvec(gpu, up(gpu, c, tiled=True), c["x"])
    assert orc.rel_l2(yr, yt) < 1e-6
    assert orc.rel_l2(yt, orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"])) < TOL


def test_repack_layout(gpu, orc):
    """Tiled word ((T*G + g)*64 + lane)*(gs/32) + 2*st + h holds qweight
    [g*gs/8 + 8*st + 2*(lane//16) + h][16*T + lane%16] (columns clamped)."""
    K, N, gs = 512, 40, 128
    c = orc.gptq_case(3, K, N, gs)
    w = up(gpu, c, tiled=True)
    got = w.qweight.cpu().numpy().view(np.uint32)
    G, T, wpl = K // gs, (N + 15) // 16, gs // 32
    assert got.size == T * 16 * K // 8
    exp = np.empty_like(got)
    for t in range(T):
        for g in range(G):
            for lane in range(64):
                for j in range(wpl):
                    pr = g * gs // 8 + 8 * (j // 2) + 2 * (lane // 16) + (j % 2)
                    exp[((t * G + g) * 64 + lane) * wpl + j] = c["qweight"][pr, min(16 * t + lane % 16, N - 1)]
    assert np.array_equal(got, exp)


def test_graph_replay_matches_eager(gpu, orc):
    """Captured decode kernels replayed several times, with eager work and
    syncs in between, give the eager result every time (no state carried
    between launches)."""
    K, N = 4096, 1024
    c = orc.gptq_case(95, K, N, 128)
    w = up(gpu, c)
    cu = orc.gptq_case(96, K, N, 128)
    wu = up(gpu, cu)
    x = torch.from_numpy(c["x"]).cuda()
    y_eager = torch.empty(1, N, device="cuda")
    y2_eager = torch.empty(1, N, device="cuda")
    M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y_eager, K, N, 128, flags=w.flags)
    M.fused_gate_up_silu(gpu, x, w.qweight, w.scales, wu.qweight, wu.scales, y2_eager, K, N, 128, flags=w.flags)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    y = torch.zeros(1, N, device="cuda")
    y2 = torch.zeros(1, N, device="cuda")
    with torch.cuda.stream(s):
        M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y, K, N, 128, flags=w.flags)  # warm on s
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y, K, N, 128, flags=w.flags)
            M.fused_gate_up_silu(gpu, x, w.qweight, w.scales, wu.qweight, wu.scales, y2, K, N, 128, flags=w.flags)
    for rep in range(4):
        y.fill_(float("nan"))
        y2.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager), rep
        assert torch.equal(y2, y2_eager), rep
        M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y_eager, K, N, 128, flags=w.flags)  # eager work between
        torch.cuda.synchronize()


@pytest.mark.parametrize("tiled", [True, False])
def test_concatenated_linears_equal_separate_calls(gpu, orc, tiled):
    """GptqWeight.cat (q/k/v sharing x): one matvec on the concatenation
    returns the separate matvecs' outputs side by side. Every group's value
    is the same exact integer sum rounded once; only the order of the f32
    additions across groups may differ (a workgroup's K split depends on how
    many tiles it owns), so they agree to f32 rounding, and both meet the
    oracle."""
    K = 1024
    cs = [orc.gptq_case(70 + i, K, n, 128, zeros=True) for i, n in enumerate((256, 64, 72))]
    ws = [up(gpu, c, tiled=tiled) for c in cs]
    x = np.ascontiguousarray(orc.gptq_case(80, K, 16, 128, M=3)["x"])
    sep = [run_matvec(gpu, w, x) for w in ws]
    cat = sta.GptqWeight.cat(ws)
    assert cat.N == 392
    y = run_matvec(gpu, cat, x)
    ysep = np.concatenate(sep, axis=1)
    assert orc.rel_l2(y, ysep) < 1e-6
    ref = np.concatenate([orc.gptq_matvec_f64(x, c["qweight"], c["scales"], K, n, 128, qzeros=c["qzeros"])
                          for c, n in zip(cs, (256, 64, 72))], axis=1)
    assert orc.rel_l2(y, ref) < TOL
    with pytest.raises(ValueError):
        sta.GptqWeight.cat([ws[2], ws[0]])  # N = 72 is not a multiple of 16 before the last part


@pytest.mark.parametrize("K,N,gs,zeros,act", [
    (4096, 8200, 128, True, True),      # 513 tiles: 2-3 tiles per workgroup, ragged last tile
    (2048, 16392, 64, True, False),     # 1025 tiles: 4 tiles per workgroup, grid beyond the CUs
    (2560, 12296, 256, False, False),   # 769 tiles
    (1024, 4104, 128, False, True),     # 257 tiles: just past one tile per CU
])
def test_multi_tile_workgroups(gpu, orc, K, N, gs, zeros, act, tune):
    """N above 16 columns per CU: one workgroup owns several 16-column tiles
    and stages x once for them. Same values as one tile per workgroup (up to
    f32 summation order across K slices) and the f64 oracle."""
    c = orc.gptq_case(K // 64 + N, K, N, gs, zeros=zeros, act_order=act)
    w = up(gpu, c)
    y = run_matvec(gpu, w, c["x"])[0]
    tune(ONE_TILE=1)
    y1 = run_matvec(gpu, w, c["x"])[0]
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
    e, e1 = orc.rel_l2(y, ref), orc.rel_l2(y, y1)
    print(f"multi-tile K={K} N={N} gs={gs}: rel-L2 {e:.3e}, vs one tile per workgroup {e1:.3e}")
    assert e < TOL and e1 < 1e-6
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("N", [11008, 8200])
def test_gate_up_multi_tile_with_zeros(gpu, orc, N):
    K, gs = 4096, 128
    cg = orc.gptq_case(73, K, N, gs, zeros=True)
    cu = orc.gptq_case(74, K, N, gs, zeros=True)
    wg_, wu_ = up(gpu, cg), up(gpu, cu)
    x = torch.from_numpy(cg["x"]).cuda()
    y = torch.empty(1, N, device="cuda")
    M.fused_gate_up_silu(gpu, x, wg_.qweight, wg_.scales, wu_.qweight, wu_.scales, y, K, N, gs,
                         gate_qz=wg_.qzeros, up_qz=wu_.qzeros, flags=wg_.flags)
    torch.cuda.synchronize()
    g = orc.gptq_matvec_f64(cg["x"], cg["qweight"], cg["scales"], K, N, gs, qzeros=cg["qzeros"])
    u = orc.gptq_matvec_f64(cg["x"], cu["qweight"], cu["scales"], K, N, gs, qzeros=cu["qzeros"])
    assert orc.rel_l2(y.cpu().numpy()[0], orc.silu_gate_f64(g, u)) < TOL


@pytest.mark.parametrize("K,N,gs,Mr,zeros,act", [
    (2048, 8200, 128, 6, True, True),     # 513 tiles, 3 per workgroup: chunks of 10 groups (10 + 6)
    (4096, 4104, 64, 13, False, False),   # 257 tiles, 2 per workgroup
    (2560, 16392, 256, 16, True, False),  # 1025 tiles, 4 per workgroup: chunks of 8 groups (8 + 2)
    (5120, 13824, 128, 8, False, True),   # configs[2]-sized GPTQ, two token blocks
])
def test_multi_token_chunked(gpu, orc, K, N, gs, Mr, zeros, act, tune):
    """Several token blocks on a multi-tile grid: x staged cooperatively in K
    chunks once per CU. Same values as the per-wave fallback (up to f32
    summation order) and the f64 oracle, every token row."""
    c = orc.gptq_case(K // 32 + N + Mr, K, N, gs, zeros=zeros, act_order=act, M=Mr)
    w = up(gpu, c)
    y = run_matvec(gpu, w, c["x"])
    tune(NO_CHUNK=1)
    y0 = run_matvec(gpu, w, c["x"])
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
    e, e0 = orc.rel_l2(y, ref), orc.rel_l2(y, y0)
    print(f"chunked K={K} N={N} gs={gs} M={Mr}: rel-L2 {e:.3e}, vs fallback {e0:.3e}")
    assert e < TOL and e0 < 1e-6
    for m in range(Mr):
        assert orc.rel_l2(y[m], ref[m]) < TOL


def test_gate_up_multi_token_chunked_with_zeros(gpu, orc):
    K, N, gs, Mr = 4096, 11008, 128, 7
    cg = orc.gptq_case(75, K, N, gs, zeros=True, M=Mr)
    cu = orc.gptq_case(76, K, N, gs, zeros=True)
    wg_, wu_ = up(gpu, cg), up(gpu, cu)
    x = torch.from_numpy(cg["x"]).cuda()
    y = torch.empty(Mr, N, device="cuda")
    M.fused_gate_up_silu(gpu, x, wg_.qweight, wg_.scales, wu_.qweight, wu_.scales, y, K, N, gs,
                         gate_qz=wg_.qzeros, up_qz=wu_.qzeros, flags=wg_.flags)
    torch.cuda.synchronize()
    g = orc.gptq_matvec_f64(cg["x"], cg["qweight"], cg["scales"], K, N, gs, qzeros=cg["qzeros"])
    u = orc.gptq_matvec_f64(cg["x"], cu["qweight"], cu["scales"], K, N, gs, qzeros=cu["qzeros"])
    ref = orc.silu_gate_f64(g, u)
    y = y.cpu().numpy()
    assert orc.rel_l2(y, ref) < TOL
    for m in range(Mr):
        assert orc.rel_l2(y[m], ref[m]) < TOL


def test_int8_repack_layout(gpu, orc):
    """st_int8_repack: tile T, group u, lane (q, c) holds bytes k = 128 u +
    16 q + 64 st + j of row 16 T + c (rows past N repeat row N - 1)."""
    K, N = 384, 40
    c = orc.int8_case(83, K, N)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
    got = w.w.cpu().numpy().reshape(3, K // 128, 64, 2, 16)  # [tile][group][lane][st][16 bytes]
    src = np.asarray(c["w"], np.int8)
    for T in range(3):
        for u in range(K // 128):
            for lane in range(64):
                n = min(16 * T + lane % 16, N - 1)
                for st in range(2):
                    k0 = 128 * u + 16 * (lane // 16) + 64 * st
                    assert np.array_equal(got[T, u, lane, st], src[n, k0:k0 + 16])


@pytest.mark.parametrize("Mr", [1, 3, 8, 16, 32])
def test_int8_tiled_equals_row_major(gpu, orc, Mr, tune):
    """Tiled and row-major INT8 weights give the same y bit for bit through
    the integer-limb kernels (the same integer products in the same order),
    within the bar of the f64 oracle. (Several f16 tokens on tiled weights
    normally take the f16-MFMA kernel; it is switched off here.)"""
    tune(I8MM_MIN_M=99)
    K, N = 5120, 4104
    c = orc.int8_case(84 + Mr, K, N, M=Mr)
    x = torch.from_numpy(c["x"]).cuda()
    ys = []
    for tiled in (True, False):
        w = sta.Int8Weight.upload(gpu, c["w"], c["scale"], tiled=tiled)
        y = torch.empty(Mr, N, device="cuda")
        M.int8_matvec(gpu, x, w.w, w.scale, y, K, N, w.flags)
        torch.cuda.synchronize()
        ys.append(y.cpu().numpy())
    assert np.array_equal(ys[0], ys[1])
    assert orc.rel_l2(ys[0], orc.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)) < TOL


@pytest.mark.parametrize("K,N,zeros,act,silu", [
    (11008, 4096, False, False, False),  # Llama-7B down: one tile per CU, 86 groups
    (9728, 2560, True, False, False),    # configs[4] down, zeros
    (11008, 1000, True, True, False),    # ragged N, act-order
    (11008, 4096, False, False, True),   # the silu(a) * b form
])
def test_two_tokens_long_k(gpu, orc, K, N, zeros, act, silu, tune):
    """Two tokens on a long K with at most one tile per CU take the one-tile
    cooperative kernel (the K-split kernel only when that does not fit): its
    y against the f64 oracle, and against the K-split kernel (forced by
    switching the cooperative kernels off)."""
    Mr, gs = 2, 128
    c = orc.gptq_case(410 + N % 97, K, N, gs, zeros=zeros, act_order=act, M=Mr)
    w = up(gpu, c)
    if silu:
        b = np.random.default_rng(5).standard_normal((Mr, K)).astype(np.float32)
        h = c["x"] / (1.0 + np.exp(-c["x"].astype(np.float64))) * b
        ref = orc.gptq_matvec_f64(h, c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])

        def run():
            xa = torch.from_numpy(c["x"]).to(gpu.device)
            xb = torch.from_numpy(b).to(gpu.device)
            y = torch.empty(Mr, N, device=gpu.device)
            M.fused_silu_gptq_down(gpu, xa, xb, w.qweight, w.scales, y, K, N, gs, w.qzeros, w.perm, w.flags)
            torch.cuda.synchronize()
            return y.cpu().numpy()
    else:
        ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
        run = lambda: run_matvec(gpu, w, c["x"])
    y = run()
    tune(NO_COOP=1)
    y_split = run()
    print(f"two tokens K={K} N={N}: rel-L2 {orc.rel_l2(y, ref):.3e} (split {orc.rel_l2(y_split, ref):.3e})")
    assert orc.rel_l2(y, ref) < TOL and orc.rel_l2(y_split, ref) < TOL
    assert orc.rel_l2(y, y_split) < 1e-6


@pytest.mark.parametrize("kind,K,N,Mr", [
    ("gptq", 9728, 2560, 16),   # configs[4] down at batch 16: 160 tiles, K split 6 ways
    ("gptq", 4096, 520, 5),     # 33 tiles, ragged
    ("dual", 2560, 1032, 12),   # gate/up with zeros
    ("int8", 5120, 1024, 8),
])
def test_multi_token_split_k(gpu, orc, kind, K, N, Mr, tune):
    """Fewer 16-column tiles than CUs, several tokens: K is split across
    workgroups (f32 partials in the workspace; the last slice of each tile
    group to finish adds them in slice order and applies the epilogue, bit
    for bit what a separate reduce kernel gives, call after call). Same
    values as without the split and as the
    per-wave fallback, up to f32 summation order; the f64 oracle's bar."""
    def run():
        y = torch.empty(Mr, N, device="cuda")
        if kind == "int8":
            M.int8_matvec(gpu, x, w.w, w.scale, y, K, N, w.flags)
        elif kind == "dual":
            M.fused_gate_up_silu(gpu, x, w.qweight, w.scales, w2.qweight, w2.scales, y, K, N, 128,
                                 gate_qz=w.qzeros, up_qz=w2.qzeros, flags=w.flags)
        else:
            M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y, K, N, 128, w.qzeros, w.perm, w.flags)
        torch.cuda.synchronize()
        return y.cpu().numpy()

    if kind == "int8":
        c = orc.int8_case(100 + Mr, K, N, M=Mr)
        w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
        ref = orc.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)
    else:
        c = orc.gptq_case(100 + Mr, K, N, 128, zeros=True, act_order=(kind == "gptq"), M=Mr)
        w = up(gpu, c)
        ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, 128, qzeros=c["qzeros"], g_idx=c["g_idx"])
        if kind == "dual":
            c2 = orc.gptq_case(200 + Mr, K, N, 128, zeros=True)
            w2 = up(gpu, c2)
            u = orc.gptq_matvec_f64(c["x"], c2["qweight"], c2["scales"], K, N, 128, qzeros=c2["qzeros"])
            ref = orc.silu_gate_f64(ref, u)
    x = torch.from_numpy(c["x"]).cuda()
    y = run()
    tune(SPLIT_REDUCE_KERNEL=0)  # the reduction fused (the default up to 8 tokens)
    y_fused = run()
    y_again = run()  # the fused reduction's counters cleared themselves
    tune(SPLIT_REDUCE_KERNEL=1)  # the same slices reduced by a kernel of their own: same order, same bits
    y_kernel = run()
    tune(SPLIT_REDUCE_KERNEL=-1)
    assert np.array_equal(y_fused, y_again) and np.array_equal(y_fused, y_kernel) and np.array_equal(y, y_kernel)
    tune(NO_KSPLIT=1)
    y1 = run()
    tune(NO_CHUNK=1)
    y0 = run()
    e = orc.rel_l2(y, ref)
    print(f"split-K {kind} K={K} N={N} M={Mr}: rel-L2 {e:.3e}, vs unsplit {orc.rel_l2(y, y1):.3e}, vs fallback {orc.rel_l2(y, y0):.3e}")
    assert e < TOL and orc.rel_l2(y, y1) < 1e-6 and orc.rel_l2(y, y0) < 1e-6
    for m in range(Mr):
        assert orc.rel_l2(y[m], ref[m]) < TOL


def test_graph_replay_multi_token_split_k(gpu, orc):
    """A captured multi-token call on a narrow linear (split-K partials in the
    context workspace + reduce) and a multi-tile chunked call, replayed with a
    different eager call that also uses the workspace in between: every replay
    gives the eager result."""
    Mr = 16
    cd = orc.gptq_case(97, 9728, 2560, 128, M=Mr)       # 160 tiles: split K
    wd = up(gpu, cd)
    cq = orc.gptq_case(98, 2560, 8200, 128, M=Mr)       # 513 tiles: chunked, no split
    wq = up(gpu, cq)
    xd = torch.from_numpy(cd["x"]).cuda()
    xq = torch.from_numpy(cq["x"]).cuda()
    co = orc.gptq_case(99, 4096, 1032, 128, M=8)        # other split-K work between replays
    wo = up(gpu, co)
    xo = torch.from_numpy(co["x"]).cuda()
    yo = torch.empty(8, 1032, device="cuda")

    def calls(yd, yq):
        M.gptq_matvec(gpu, "d", xd, wd.qweight, wd.scales, yd, 9728, 2560, 128, flags=wd.flags)
        M.gptq_matvec(gpu, "q", xq, wq.qweight, wq.scales, yq, 2560, 8200, 128, flags=wq.flags)

    yd_e = torch.empty(Mr, 2560, device="cuda")
    yq_e = torch.empty(Mr, 8200, device="cuda")
    calls(yd_e, yq_e)
    torch.cuda.synchronize()
    yd = torch.zeros_like(yd_e)
    yq = torch.zeros_like(yq_e)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        calls(yd, yq)  # warm on s
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            calls(yd, yq)
    for rep in range(4):
        yd.fill_(float("nan"))
        yq.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yd, yd_e), rep
        assert torch.equal(yq, yq_e), rep
        M.gptq_matvec(gpu, "o", xo, wo.qweight, wo.scales, yo, 4096, 1032, 128, flags=wo.flags)
        torch.cuda.synchronize()
    ref = orc.gptq_matvec_f64(cd["x"], cd["qweight"], cd["scales"], 9728, 2560, 128)
    assert orc.rel_l2(yd.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("mode", ["1", "2"])
@pytest.mark.parametrize("K,N,gs,Mr,zeros,act", [
    (4096, 4096, 128, 1, False, False),   # q_proj shape, one tile per workgroup
    (11008, 4104, 128, 1, True, True),    # long K, ragged
    (4096, 11008, 64, 3, False, False),   # multi-tile, three tokens
    (2560, 1024, 256, 1, True, False),
])
def test_staging_modes_agree(gpu, orc, mode, K, N, gs, Mr, zeros, act, tune):
    """The single-block cooperative kernels forced into each staging mode
    (1: staging waves, 2: every wave stages its own groups) meet the oracle's
    bar and agree with the launcher's own choice up to f32 summation order."""
    c = orc.gptq_case(K // 16 + N + Mr, K, N, gs, zeros=zeros, act_order=act, M=Mr)
    w = up(gpu, c)
    y_auto = run_matvec(gpu, w, c["x"])
    tune(STAGE_MODE=int(mode))
    y = run_matvec(gpu, w, c["x"])
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
    assert orc.rel_l2(y, ref) < TOL
    assert orc.rel_l2(y, y_auto) < 1e-6


@pytest.mark.parametrize("tiled", [True, False])
def test_linear_dispatch_int8_honours_layout(gpu, orc, tiled):
    """linear() on an Int8Weight passes the weight's layout flag (tiled by
    default at upload)."""
    K, N, Mr = 1024, 520, 3
    c = orc.int8_case(110, K, N, M=Mr)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"], tiled=tiled)
    y = torch.empty(Mr, N, device="cuda")
    sta.linear(gpu, torch.from_numpy(c["x"]).cuda(), w, y)
    torch.cuda.synchronize()
    assert orc.rel_l2(y.cpu().numpy(), orc.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)) < TOL


@pytest.mark.parametrize("K,gs,Mr", [(32768, 128, 1), (16384, 64, 5), (24576, 256, 1)])
def test_long_k(gpu, orc, K, gs, Mr):
    """K at the largest sizes the entry points take (up to 32768): the
    launcher's path for long K (LDS limits the cooperative staging)."""
    N = 264
    c = orc.gptq_case(K // 1024 + Mr, K, N, gs, zeros=True, act_order=True, M=Mr)
    w = up(gpu, c)
    y = run_matvec(gpu, w, c["x"])
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
    assert orc.rel_l2(y, ref) < TOL


@pytest.mark.parametrize("Mr,K,N", [
    (2, 128, 20),       # one group, one partial chunk, two tiles
    (5, 384, 36),       # ragged N, partial chunk
    (16, 1152, 264),    # one 16-row block, a chunk and a bit
    (17, 5120, 1000),   # two row blocks, 63 tiles (one per workgroup)
    (32, 2176, 4104),   # 257 tiles: one or two per workgroup
    (8, 256, 24576),    # 1536 tiles: six per workgroup, two waves per tile
    (3, 256, 36880),    # 2305 tiles: more than eight per CU, more workgroups than CUs
])
def test_int8_mm_f16(gpu, orc, Mr, K, N, tune):
    """Several f16 tokens on tiled INT8 weights: the f16-MFMA kernel (every
    int8 weight and f16 x exact in f16, products exact in f32, f32 sums)
    against the f64 oracle, and against the integer-limb kernels."""
    c = orc.int8_case(120 + Mr, K, N, M=Mr)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
    x = torch.from_numpy(c["x"]).cuda()

    def run():
        y = torch.full((Mr, N), float("nan"), device="cuda")
        M.int8_matvec(gpu, x, w.w, w.scale, y, K, N, w.flags)
        torch.cuda.synchronize()
        return y.cpu().numpy()

    y = run()
    ref = orc.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)
    e = orc.rel_l2(y, ref)
    print(f"int8 f16-MFMA M={Mr} K={K} N={N} rel-L2 {e:.3e}")
    assert np.isfinite(y).all() and e < 1e-6  # f32 summation error only
    tune(I8MM_MIN_M=99)
    assert orc.rel_l2(run(), ref) < TOL


def test_int8_mm_f16_integer_exact(gpu, orc):
    """Integer x (|x| <= 4) and unit scales: every partial sum is an integer
    below 2^24, so the f16-MFMA kernel's y equals the exact integer product
    bit for bit."""
    Mr, K, N = 32, 3072, 520
    rng = np.random.default_rng(7)
    wq = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    xi = rng.integers(-4, 5, size=(Mr, K)).astype(np.float16)
    w = sta.Int8Weight.upload(gpu, wq, np.ones(N, np.float32))
    y = torch.empty(Mr, N, device="cuda")
    M.int8_matvec(gpu, torch.from_numpy(xi).cuda(), w.w, w.scale, y, K, N, w.flags)
    torch.cuda.synchronize()
    exact = xi.astype(np.int64) @ wq.astype(np.int64).T
    assert np.array_equal(y.cpu().numpy(), exact.astype(np.float32))


def test_int8_mm_f16_graph_replay(gpu, orc):
    """The f16-MFMA kernel under graph capture: every replay equals the eager
    result bit for bit (no workspace, no memset)."""
    Mr, K, N = 24, 1280, 1040
    c = orc.int8_case(140, K, N, M=Mr)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
    x = torch.from_numpy(c["x"]).cuda()
    y = torch.empty(Mr, N, device="cuda")
    M.int8_matvec(gpu, x, w.w, w.scale, y, K, N, w.flags)
    torch.cuda.synchronize()
    eager = y.clone()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            M.int8_matvec(gpu, x, w.w, w.scale, y, K, N, w.flags)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)


def _force_i4mm(tune):
    tune(I4MM_MIN_M=2)
    tune(I4MM_MIN_TILES=1)


def _gate_up(gpu, wg, wu, x, dtype=torch.float32):
    xt = torch.from_numpy(np.ascontiguousarray(x)).to(gpu.device)
    if dtype == torch.float16:
        xt = xt.half()
    y = torch.empty(x.shape[0], wg.N, device=gpu.device)
    M.fused_gate_up_silu(gpu, xt, wg.qweight, wg.scales, wu.qweight, wu.scales, y, wg.K, wg.N, wg.group_size,
                         gate_qz=wg.qzeros, up_qz=wu.qzeros, perm=wg.perm, flags=wg.flags)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("Mr,K,N,gs,zeros,f16,dual", [
    (2, 128, 64, 128, False, False, False),     # one unit, one tile
    (5, 384, 72, 64, True, False, False),       # group 64, ragged last tile
    (16, 2560, 6144, 128, False, False, False),  # configs[4] q|k|v at batch 16
    (16, 9728, 2560, 128, False, False, False),  # configs[4] down: 160 tiles, 76 units
    (9, 4096, 520, 256, True, False, False),    # group 256, two 16-row blocks
    (12, 1024, 1000, 128, True, True, False),   # f16 x
    (3, 256, 36880, 128, False, False, False),  # 2305 tiles: more workgroups than CUs
    (16, 2560, 9728, 128, False, False, True),  # configs[4] gate/up at batch 16
    (6, 1536, 776, 64, True, True, True),       # gate/up, f16 x, zeros, group 64
])
def test_int4_mm_f16(gpu, orc, Mr, K, N, gs, zeros, f16, dual, tune):
    """2..16 tokens on tiled GPTQ weights: the f16-MFMA kernel ((q - z)
    exact in f16, f32 x as two f16 rows per 128-k block scaled by a power of
    two, exact products, f32 sums and per-group scaling) against the f64
    oracle, and against the integer-limb kernels. (The entry points choose
    it for 12+ tokens and more tiles than CUs; forced here.)"""
    _force_i4mm(tune)
    xd = np.float16 if f16 else np.float32
    c = orc.gptq_case(150 + Mr, K, N, gs, zeros=zeros, M=Mr, x_dtype=xd)
    w = up(gpu, c)
    dt = torch.float16 if f16 else torch.float32
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"])
    if dual:
        c2 = orc.gptq_case(250 + Mr, K, N, gs, zeros=zeros)
        w2 = up(gpu, c2)
        ref = orc.silu_gate_f64(ref, orc.gptq_matvec_f64(c["x"], c2["qweight"], c2["scales"], K, N, gs,
                                                         qzeros=c2["qzeros"]))
        run = lambda: _gate_up(gpu, w, w2, c["x"], dt)
    else:
        run = lambda: run_matvec(gpu, w, c["x"], dt)
    y = run()
    e = orc.rel_l2(y, ref)
    print(f"int4 f16-MFMA M={Mr} K={K} N={N} gs={gs} dual={dual} rel-L2 {e:.3e}")
    assert np.isfinite(y).all() and e < 1e-5
    tune(I4MM_MIN_M=99)
    assert orc.rel_l2(run(), ref) < TOL


@pytest.mark.parametrize("Mr,K,N,gs,zeros,dual", [
    (2, 128, 64, 128, False, False),       # one unit, one tile
    (5, 384, 72, 64, True, False),         # group 64, ragged last tile
    (16, 2560, 6144, 128, False, False),   # configs[4] q|k|v at batch 16
    (9, 4096, 520, 256, True, False),      # group 256, two 16-row blocks
    (3, 256, 36880, 128, False, False),    # more workgroups than CUs
    (16, 2560, 9728, 128, False, True),    # configs[4] gate/up at batch 16
    (6, 1536, 776, 64, True, True),        # gate/up, zeros, group 64
])
def test_int4_mm_f16_split_in_kernel(gpu, orc, Mr, K, N, gs, zeros, dual, tune):
    """f32 x on the f16-MFMA kernel is split into its hi / lo f16 rows and
    per-unit power-of-two factors inside the kernel, at staging (no
    pre-pass launch): the same arithmetic as the pre-pass, so y equals the
    pre-pass path (I4MM_PREPASS=1) bit for bit, and the f64 oracle within
    1e-5. x spans large and tiny magnitudes (per-unit exponents differ)."""
    _force_i4mm(tune)
    c = orc.gptq_case(330 + Mr, K, N, gs, zeros=zeros, M=Mr)
    x = c["x"].copy()
    x[:, : K // 2] *= np.float32(3e4)
    x[:, K // 2:] *= np.float32(1e-3)
    x[0, :128] = 0.0  # an all-zero unit: factor 1
    w = up(gpu, c)
    ref = orc.gptq_matvec_f64(x, c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"])
    if dual:
        c2 = orc.gptq_case(340 + Mr, K, N, gs, zeros=zeros)
        w2 = up(gpu, c2)
        ref = orc.silu_gate_f64(ref, orc.gptq_matvec_f64(x, c2["qweight"], c2["scales"], K, N, gs, qzeros=c2["qzeros"]))
        run = lambda: _gate_up(gpu, w, w2, x)
    else:
        run = lambda: run_matvec(gpu, w, x, torch.float32)
    y_in = run()
    tune(I4MM_PREPASS=1)
    y_pre = run()
    np.testing.assert_array_equal(y_in, y_pre)
    e = orc.rel_l2(y_in, ref)
    print(f"int4 f16-MFMA in-kernel split M={Mr} K={K} N={N} gs={gs} dual={dual} rel-L2 {e:.3e}")
    assert np.isfinite(y_in).all() and e < 1e-5


@pytest.mark.parametrize("Mr,K,N,gs,zeros,f16,dual", [
    (16, 2560, 9728, 128, False, False, True),   # configs[4] gate/up: 608 tile pairs, 3 per workgroup
    (9, 1024, 11008, 128, True, True, True),     # Llama-7B gate/up width, f16 x, zeros
    (12, 1024, 12288, 128, False, False, False),  # one source, 768 tiles: 3 per workgroup, 4 waves each
    (16, 1024, 20480, 64, True, False, False),   # one source, 1280 tiles: 5 per workgroup, group 64
    (11, 2048, 9728, 256, True, True, True),     # gate/up, group 256, f16 x, zeros
])
def test_int4_mm_f16_12_waves(gpu, orc, Mr, K, N, gs, zeros, f16, dual, tune):
    """Workgroups whose tiles use at most 12 waves launch 12 (the idle waves
    of a 16-wave workgroup would still issue the loop's VALU work): same
    per-wave work and reduction order, so with one source per wave the
    result equals the 16-wave launch bit for bit. Gate/up by default gives
    a wave both sources of its tile (I4MM_PAIR): 4-way instead of 2-way K
    slices, so its sums round differently; it is held to the f64 oracle
    (1e-5), like the one-source forms."""
    _force_i4mm(tune)
    xd = np.float16 if f16 else np.float32
    c = orc.gptq_case(190 + Mr, K, N, gs, zeros=zeros, M=Mr, x_dtype=xd)
    w = up(gpu, c)
    dt = torch.float16 if f16 else torch.float32
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"])
    if dual:
        c2 = orc.gptq_case(290 + Mr, K, N, gs, zeros=zeros)
        w2 = up(gpu, c2)
        ref = orc.silu_gate_f64(ref, orc.gptq_matvec_f64(c["x"], c2["qweight"], c2["scales"], K, N, gs,
                                                         qzeros=c2["qzeros"]))
        run = lambda: _gate_up(gpu, w, w2, c["x"], dt)
    else:
        run = lambda: run_matvec(gpu, w, c["x"], dt)
    yd = run()
    tune(I4MM_PAIR=0)
    y12 = run()
    tune(I4MM_WAVES=16)
    y16 = run()
    for name, y in (("default", yd), ("one source per wave", y12)):
        e = orc.rel_l2(y, ref)
        print(f"int4 f16-MFMA 12 waves ({name}) M={Mr} K={K} N={N} gs={gs} dual={dual} rel-L2 {e:.3e}")
        assert np.isfinite(y).all() and e < 1e-5
    assert np.array_equal(y12, y16)


@pytest.mark.parametrize("Mr,K,N,gs,zeros,f16,dual", [
    (16, 2560, 6144, 128, False, False, False),  # configs[4] q|k|v shape, f32 x (gathered in the pre-pass)
    (12, 1024, 4112, 64, True, True, False),     # f16 x (gather pass), zeros, group 64, 257 tiles
    (16, 2560, 9728, 128, True, False, True),    # gate/up, f32 x
    (13, 1536, 5200, 256, False, True, True),    # gate/up, f16 x, group 256
])
def test_int4_mm_f16_act_order(gpu, orc, Mr, K, N, gs, zeros, f16, dual, tune):
    """Act-order checkpoints on the f16-MFMA kernel (9-16 tokens): x read
    through the upload's permutation (rows sorted by group), against the f64
    oracle with scale[g_idx[k]], and against the integer-limb kernels."""
    _force_i4mm(tune)
    xd = np.float16 if f16 else np.float32
    c = orc.gptq_case(170 + Mr, K, N, gs, zeros=zeros, act_order=True, M=Mr, x_dtype=xd)
    w = up(gpu, c)
    assert w.perm is not None
    dt = torch.float16 if f16 else torch.float32
    f64 = lambda cc: orc.gptq_matvec_f64(c["x"], cc["qweight"], cc["scales"], K, N, gs, qzeros=cc["qzeros"],
                                         g_idx=c["g_idx"])
    ref = f64(c)
    if dual:
        c2 = orc.gptq_case(270 + Mr, K, N, gs, zeros=zeros)
        c2["g_idx"] = c["g_idx"]
        w2 = up(gpu, c2)
        ref = orc.silu_gate_f64(ref, f64(c2))
        run = lambda: _gate_up(gpu, w, w2, c["x"], dt)
    else:
        run = lambda: run_matvec(gpu, w, c["x"], dt)
    y = run()
    e = orc.rel_l2(y, ref)
    print(f"int4 f16-MFMA act-order M={Mr} K={K} N={N} gs={gs} dual={dual} rel-L2 {e:.3e}")
    assert np.isfinite(y).all() and e < 1e-5
    tune(I4MM_MIN_M=99)
    assert orc.rel_l2(run(), ref) < TOL


@pytest.mark.parametrize("Mr,N,dual,want", [
    (5, 4112, False, True),     # 257 tiles, 5 tokens: the f16-MFMA kernel
    (11, 4112, True, True),     # gate/up at 11 tokens
    (6, 4112, True, True),      # gate/up at 6 tokens
    (4, 4112, False, False),    # 4 tokens: the limb (or streaming) kernels
    (10, 4096, False, True),    # 256 tiles, not more than the CUs: groups of 8 tiles, K split across workgroups
    (8, 4096, False, False),    # 8 tokens on 256 tiles: the limb kernels
])
def test_int4_mm_f16_default_routing(gpu, orc, Mr, N, dual, want, tune):
    """Which kernel the GPTQ entry points pick by default on an MI355X (256
    CUs): the f16-MFMA kernel from 5 tokens on linears with more 16-column
    tiles than CUs and from 9 tokens on the others (with K split across
    workgroups), the integer-limb kernels below. The default call's y
    must equal, bit for bit, the call with that kernel forced; both are
    checked against the f64 oracle."""
    ncu = torch.cuda.get_device_properties(gpu.device).multi_processor_count
    if ncu != 256:
        pytest.skip(f"routing thresholds are stated for 256 CUs, this GPU has {ncu}")
    K, gs = 1024, 128
    c = orc.gptq_case(190 + Mr, K, N, gs, zeros=True, M=Mr)
    w = up(gpu, c)
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"])
    if dual:
        c2 = orc.gptq_case(290 + Mr, K, N, gs, zeros=True)
        w2 = up(gpu, c2)
        ref = orc.silu_gate_f64(ref, orc.gptq_matvec_f64(c["x"], c2["qweight"], c2["scales"], K, N, gs,
                                                         qzeros=c2["qzeros"]))
        run = lambda: _gate_up(gpu, w, w2, c["x"])
    else:
        run = lambda: run_matvec(gpu, w, c["x"], torch.float32)
    y = run()
    if want:
        _force_i4mm(tune)
    else:
        tune(I4MM_MIN_M=99)
    y_forced = run()
    assert orc.rel_l2(y, ref) < TOL
    np.testing.assert_array_equal(y, y_forced)


@pytest.mark.parametrize("Mr,K,N,gs,zeros,f16,dual,act", [
    (16, 4096, 2560, 128, False, False, False, False),  # configs[4] o: 160 tiles, 20 groups of 8, 12 K slices
    (16, 9728, 2560, 128, False, False, False, False),  # configs[4] down: 76 units
    (9, 11008, 4096, 128, True, False, False, False),   # Llama-7B down at 9 tokens, zeros
    (12, 4096, 4096, 128, False, True, False, False),   # f16 x, 256 tiles
    (10, 2048, 520, 64, True, False, False, False),     # group 64, ragged last tile
    (13, 3072, 776, 256, False, False, False, False),   # group 256
    (16, 2560, 1024, 128, False, False, True, False),   # gate/up on 64 tile pairs
    (11, 1536, 776, 128, True, True, True, False),      # gate/up, f16 x, zeros
    (16, 4096, 2560, 128, True, False, False, True),    # act-order, f32 x: pre-pass rows, then the partials
    (14, 2048, 1040, 128, False, True, True, True),     # act-order, f16 x gathered, gate/up
])
def test_int4_mm_f16_k_split(gpu, orc, Mr, K, N, gs, zeros, f16, dual, act, tune):
    """9-16 tokens on no more 16-column tiles than CUs: the f16-MFMA kernel
    takes groups of 8 tiles with K split across workgroups (whole chunks per
    slice), f32 partial sums in the workspace (after the pre-pass rows when
    there are any) added in slice order by a reduce launch. Against the f64
    oracle (1e-5), against the integer-limb kernels, and deterministic."""
    xd = np.float16 if f16 else np.float32
    c = orc.gptq_case(400 + Mr, K, N, gs, zeros=zeros, act_order=act, M=Mr, x_dtype=xd)
    w = up(gpu, c)
    dt = torch.float16 if f16 else torch.float32
    f64 = lambda cc: orc.gptq_matvec_f64(c["x"], cc["qweight"], cc["scales"], K, N, gs, qzeros=cc["qzeros"],
                                         g_idx=c["g_idx"] if act else None)
    ref = f64(c)
    if dual:
        c2 = orc.gptq_case(410 + Mr, K, N, gs, zeros=zeros)
        if act:
            c2["g_idx"] = c["g_idx"]
        w2 = up(gpu, c2)
        ref = orc.silu_gate_f64(ref, f64(c2))
        run = lambda: _gate_up(gpu, w, w2, c["x"], dt)
    else:
        run = lambda: run_matvec(gpu, w, c["x"], dt)
    tune(I4MM_MIN_M=2)
    y = run()
    e = orc.rel_l2(y, ref)
    print(f"int4 f16-MFMA K split M={Mr} K={K} N={N} gs={gs} dual={dual} act={act} rel-L2 {e:.3e}")
    assert np.isfinite(y).all() and e < 1e-5
    np.testing.assert_array_equal(run(), y)
    tune(I4MM_SPLIT_TILES=0)
    assert orc.rel_l2(run(), ref) < TOL


@pytest.mark.parametrize("Mr,K,N,gs,zeros,f16,act,dual", [
    (32, 2560, 10240, 128, False, False, False, False),  # configs[4] q|k|v at 32 tokens: 64 MFMA rows
    (17, 2048, 6160, 256, True, False, False, False),    # 17 tokens, group 256, ragged last tile
    (24, 9728, 2560, 128, True, False, False, False),    # few tiles: K split across workgroups
    (32, 1024, 8200, 128, False, True, False, False),    # f16 x: two 16-row blocks
    (20, 2048, 4160, 128, True, False, True, False),     # act-order: the pre-pass splits 20 tokens
    (32, 1024, 4160, 64, False, False, False, False),    # group 64 with f32 x: 16-token blocks
    (32, 2560, 9728, 128, False, False, False, True),    # configs[4] gate/up at 32 tokens, one source per wave
    (19, 1024, 2064, 256, True, True, True, True),       # gate/up, f16 x, act-order, zeros
])
def test_int4_mm_f16_32_tokens(gpu, orc, Mr, K, N, gs, zeros, f16, act, dual, tune):
    """17-32 tokens in one f16-MFMA launch (the weights read once; f32 x as
    64 hi/lo rows, 2-unit chunks; gate/up with one source per wave), against
    the f64 oracle (1e-5), equal to the same call in 16-token pieces on the
    integer-limb kernels within the bar, and deterministic."""
    xd = np.float16 if f16 else np.float32
    c = orc.gptq_case(430 + Mr, K, N, gs, zeros=zeros, act_order=act, M=Mr, x_dtype=xd)
    w = up(gpu, c)
    dt = torch.float16 if f16 else torch.float32
    f64 = lambda cc: orc.gptq_matvec_f64(c["x"], cc["qweight"], cc["scales"], K, N, gs, qzeros=cc["qzeros"],
                                         g_idx=c["g_idx"] if act else None)
    ref = f64(c)
    if dual:
        c2 = orc.gptq_case(440 + Mr, K, N, gs, zeros=zeros)
        if act:
            c2["g_idx"] = c["g_idx"]
        w2 = up(gpu, c2)
        ref = orc.silu_gate_f64(ref, f64(c2))
        run = lambda: _gate_up(gpu, w, w2, c["x"], dt)
    else:
        run = lambda: run_matvec(gpu, w, c["x"], dt)
    y = run()
    e = orc.rel_l2(y, ref)
    print(f"int4 f16-MFMA {Mr} tokens K={K} N={N} gs={gs} act={act} dual={dual} rel-L2 {e:.3e}")
    assert np.isfinite(y).all() and e < 1e-5
    np.testing.assert_array_equal(run(), y)
    tune(I4MM_MIN_M=99)
    assert orc.rel_l2(run(), ref) < TOL


def test_int4_mm_f16_integer_exact(gpu, orc, tune):
    """Integer x, unit scales, zeros: every product and partial sum is an
    integer below 2^24, so y equals the exact integer result bit for bit
    (pins the nibble order, the zero nibble and the row/column mapping)."""
    _force_i4mm(tune)
    Mr, K, N, gs = 11, 1152, 136, 128
    c = orc.gptq_case(170, K, N, gs, zeros=True)
    rng = np.random.default_rng(3)
    x = rng.integers(-3, 4, size=(Mr, K)).astype(np.float32)
    c["scales"] = np.ones_like(c["scales"])
    w = up(gpu, c)
    y = run_matvec(gpu, w, x)
    qw, qz = c["qweight"], c["qzeros"]
    q = np.stack([(qw >> (4 * j)) & 0xF for j in range(8)], axis=1).reshape(K, N).astype(np.int64)
    z = np.stack([(qz >> (4 * j)) & 0xF for j in range(8)], axis=2).reshape(K // gs, N).astype(np.int64)
    Wd = q - np.repeat(z, gs, axis=0)
    assert np.array_equal(y, (x.astype(np.int64) @ Wd).astype(np.float32))


def test_int4_mm_f16_wide_range_x(gpu, orc, tune):
    """f32 x spanning 1e-30 .. 1e30 across 128-k blocks (outside f16's
    range): the per-block power-of-two split keeps the bar."""
    _force_i4mm(tune)
    Mr, K, N = 7, 2048, 264
    c = orc.gptq_case(171, K, N, 128, M=Mr)
    blk = np.repeat(10.0 ** np.linspace(-30, 30, K // 128), 128).astype(np.float32)
    x = (c["x"] * blk).astype(np.float32)
    w = up(gpu, c)
    y = run_matvec(gpu, w, x)
    ref = orc.gptq_matvec_f64(x, c["qweight"], c["scales"], K, N, 128)
    assert np.isfinite(y).all() and orc.rel_l2(y, ref) < 1e-5


def test_int4_mm_f16_graph_replay(gpu, orc, tune):
    """Gate/up and matvec on the f16-MFMA kernel under graph capture: every
    replay equals the eager result bit for bit."""
    _force_i4mm(tune)
    Mr, K, N = 16, 2560, 1040
    c = orc.gptq_case(172, K, N, 128, M=Mr)
    c2 = orc.gptq_case(173, K, N, 128)
    w, w2 = up(gpu, c), up(gpu, c2)
    x = torch.from_numpy(c["x"]).cuda()
    y = torch.empty(Mr, N, device="cuda")
    h = torch.empty(Mr, N, device="cuda")

    def calls():
        M.gptq_matvec(gpu, "t", x, w.qweight, w.scales, y, K, N, 128, None, None, w.flags)
        M.fused_gate_up_silu(gpu, x, w.qweight, w.scales, w2.qweight, w2.scales, h, K, N, 128, flags=w.flags)

    calls()
    torch.cuda.synchronize()
    ye, he = y.clone(), h.clone()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            calls()
    for _ in range(3):
        y.zero_()
        h.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ye) and torch.equal(h, he)


def test_int4_mm_f16_zeros_plus_one(gpu, orc, tune):
    """AutoGPTQ-v1 zero points (stored z - 1, ST_FLAG_ZEROS_PLUS_ONE) on the
    f16-MFMA kernel, matvec and gate/up, against the f64 oracle."""
    _force_i4mm(tune)
    Mr, K, N, gs = 14, 1280, 392, 128
    c = orc.gptq_case(180, K, N, gs, zeros=True, M=Mr)
    c2 = orc.gptq_case(181, K, N, gs, zeros=True)
    w, w2 = up(gpu, c, zeros_plus_one=True), up(gpu, c2, zeros_plus_one=True)
    g = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], zero_offset=1)
    u = orc.gptq_matvec_f64(c["x"], c2["qweight"], c2["scales"], K, N, gs, qzeros=c2["qzeros"], zero_offset=1)
    assert orc.rel_l2(run_matvec(gpu, w, c["x"]), g) < 1e-5
    assert orc.rel_l2(_gate_up(gpu, w, w2, c["x"]), orc.silu_gate_f64(g, u)) < 1e-5
