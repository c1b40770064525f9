"""GPU tests of the M-token callers: the fused silu.down prefill GEMM
(st_gptq_i4_silu_gemm), DecoderLinears and DeltaNetLinears (one layer's
projections for decode and for prefill, of either kind), against the f64
oracle through the C ABI."""
import numpy as np
import pytest
import torch

import shady_thinker_amd as sta
from shady_thinker_amd import model as M

pytestmark = pytest.mark.gpu

TOL_DECODE = 1e-4   # rel-L2, f32-accumulate matvec (north_star)
TOL_GEMM = 2e-3     # rel-L2, f16-MFMA GEMM (north_star)


def up(gpu, c, tiled=True):
    return sta.GptqWeight.upload(gpu, c["qweight"], c["scales"], c["gs"], qzeros=c["qzeros"], g_idx=c["g_idx"],
                                 tiled=tiled)


def ref(orc, x, c):
    return orc.gptq_matvec_f64(x, c["qweight"], c["scales"], c["K"], c["N"], c["gs"], qzeros=c["qzeros"],
                               g_idx=c["g_idx"])


@pytest.mark.parametrize("Mr,K,N,gs,zeros,act,tiled", [
    (40, 512, 264, 128, True, True, True),
    (200, 1024, 520, 64, False, False, True),
    (33, 768, 136, 256, True, False, False),
])
def test_silu_gemm(gpu, orc, Mr, K, N, gs, zeros, act, tiled):
    """C = (silu(g) * u) . dequant(W) for a block of tokens: the reference's
    fused_silu_gptq_down, M rows at a time, against f64 (silu of the f16
    inputs, then the f64 matvec); f16 and f32 outputs."""
    c = orc.gptq_case(60 + gs, K, N, gs, zeros=zeros, act_order=act)
    rng = np.random.default_rng(Mr)
    g = rng.standard_normal((Mr, K)).astype(np.float16)
    u = rng.standard_normal((Mr, K)).astype(np.float16)
    w = up(gpu, c, tiled)
    want = ref(orc, orc.silu_gate_f64(g, u), c)
    for dt in (torch.float32, torch.float16):
        y = torch.empty(Mr, N, device="cuda", dtype=dt)
        M.fused_silu_gptq_gemm(gpu, torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda(), w.qweight, w.scales, y,
                               K, N, gs, w.qzeros, w.perm, w.flags)
        torch.cuda.synchronize()
        e = orc.rel_l2(y.float().cpu().numpy(), want)
        print(f"silu GEMM M={Mr} K={K} N={N} gs={gs} {dt}: rel-L2 {e:.3e}")
        assert e < TOL_GEMM


@pytest.mark.parametrize("split", [False, True])
def test_silu_gemm_beyond_f16_range(gpu, orc, tune, split):
    """silu(g) * u above the f16 maximum (g, u up to 6e4: h up to 3.6e9; the
    A operand is f16): those rows are scaled by a power of two in the
    pre-pass and scaled back on C, so C stays finite and within the bar of
    the f64 oracle (every row separately: small-range rows beside them are
    unaffected), with and without split-K (partials carry the scale)."""
    K, N, gs = 1024, 264, 128
    c = orc.gptq_case(62, K, N, gs, zeros=True)
    w = up(gpu, c, True)
    rng = np.random.default_rng(5)
    g = rng.standard_normal((40, K)).astype(np.float32)
    u = rng.standard_normal((40, K)).astype(np.float32)
    g[1], u[1] = g[1] * 300, u[1] * 300          # |h| around 1e5: past 65504
    g[2, :16], u[2, :16] = 60000.0, -60000.0      # a few h of -3.6e9
    g[3] = np.minimum(np.abs(g[3]) * 2e4, 6e4)     # every h large (g stays a finite f16)
    g, u = g.astype(np.float16), u.astype(np.float16)
    want = ref(orc, orc.silu_gate_f64(g, u), c)
    if not split:
        tune(GEMM_NO_SPLIT=1)
    y = torch.empty(40, N, device="cuda")
    M.fused_silu_gptq_gemm(gpu, torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda(), w.qweight, w.scales, y, K, N,
                           gs, w.qzeros, w.perm, w.flags)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert np.isfinite(y).all()
    for r in range(40):
        e = orc.rel_l2(y[r], want[r])
        assert e < TOL_GEMM, (r, e)


def test_silu_gemm_zero_gate(gpu, orc):
    """silu(0) = 0: a zero gate gives C = 0 exactly whatever up holds."""
    K, N, Mr = 512, 72, 48
    c = orc.gptq_case(61, K, N, 128)
    w = up(gpu, c)
    g = torch.zeros(Mr, K, device="cuda", dtype=torch.float16)
    u = torch.randn(Mr, K, device="cuda").half()
    y = torch.full((Mr, N), 7.0, device="cuda")
    M.fused_silu_gptq_gemm(gpu, g, u, w.qweight, w.scales, y, K, N, 128, flags=w.flags)
    torch.cuda.synchronize()
    assert torch.count_nonzero(y).item() == 0


def _layer(gpu, orc, H, Q, KV, I, gs, zeros=False):
    cs = {}
    for i, (name, k, n) in enumerate((("q", H, Q), ("k", H, KV), ("v", H, KV), ("o", Q, H), ("gate", H, I),
                                       ("up", H, I), ("down", I, H))):
        cs[name] = orc.gptq_case(300 + i, k, n, gs, zeros=zeros)
    ws = {n: up(gpu, c) for n, c in cs.items()}
    return cs, sta.DecoderLinears(ws["q"], ws["k"], ws["v"], ws["o"], ws["gate"], ws["up"], ws["down"])


@pytest.mark.parametrize("Mr", [1, 3, 20])
def test_decoder_linears_decode(gpu, orc, Mr):
    """One layer's projections for 1-32 tokens (f32): q|k|v, o, h =
    silu(x.Wg) * (x.Wu) and down on h, each against the f64 oracle."""
    H, Q, KV, I, gs = 256, 256, 128, 512, 128
    cs, layer = _layer(gpu, orc, H, Q, KV, I, gs, zeros=True)
    rng = np.random.default_rng(Mr)
    x = rng.standard_normal((Mr, H)).astype(np.float32)
    attn = rng.standard_normal((Mr, Q)).astype(np.float32)
    qkv = torch.empty(Mr, Q + 2 * KV, device="cuda")
    o = torch.empty(Mr, H, device="cuda")
    h = torch.empty(Mr, I, device="cuda")
    d = torch.empty(Mr, H, device="cuda")
    layer.decode(gpu, torch.from_numpy(x).cuda(), torch.from_numpy(attn).cuda(), qkv, o, h, d)
    torch.cuda.synchronize()
    want_qkv = np.concatenate([ref(orc, x, cs[n]) for n in ("q", "k", "v")], axis=1)
    want_h = orc.silu_gate_f64(ref(orc, x, cs["gate"]), ref(orc, x, cs["up"]))
    assert orc.rel_l2(qkv.cpu().numpy(), want_qkv) < TOL_DECODE
    assert orc.rel_l2(o.cpu().numpy(), ref(orc, attn, cs["o"])) < TOL_DECODE
    assert orc.rel_l2(h.cpu().numpy(), want_h) < TOL_DECODE
    # down on the h this call produced (f32, as the reference's chain)
    assert orc.rel_l2(d.cpu().numpy(), ref(orc, h.cpu().numpy(), cs["down"])) < TOL_DECODE


def test_decoder_linears_prefill(gpu, orc):
    """One layer's projections for a 48-token block (f16) through the GEMM:
    q|k|v, o, gate, up, and down on silu(gate) * up fused into the GEMM's A
    pass, each against the f64 oracle on the same f16 inputs."""
    H, Q, KV, I, gs, Mr = 256, 256, 128, 512, 128, 48
    cs, layer = _layer(gpu, orc, H, Q, KV, I, gs)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((Mr, H)).astype(np.float16)
    attn = rng.standard_normal((Mr, Q)).astype(np.float16)
    f16 = dict(device="cuda", dtype=torch.float16)
    qkv, o = torch.empty(Mr, Q + 2 * KV, **f16), torch.empty(Mr, H, **f16)
    g, u, d = torch.empty(Mr, I, **f16), torch.empty(Mr, I, **f16), torch.empty(Mr, H, **f16)
    layer.prefill(gpu, torch.from_numpy(x).cuda(), torch.from_numpy(attn).cuda(), qkv, o, g, u, d)
    torch.cuda.synchronize()
    want_qkv = np.concatenate([ref(orc, x, cs[n]) for n in ("q", "k", "v")], axis=1)
    assert orc.rel_l2(qkv.float().cpu().numpy(), want_qkv) < TOL_GEMM
    assert orc.rel_l2(o.float().cpu().numpy(), ref(orc, attn, cs["o"])) < TOL_GEMM
    assert orc.rel_l2(g.float().cpu().numpy(), ref(orc, x, cs["gate"])) < TOL_GEMM
    assert orc.rel_l2(u.float().cpu().numpy(), ref(orc, x, cs["up"])) < TOL_GEMM
    want_d = ref(orc, orc.silu_gate_f64(g.cpu().numpy(), u.cpu().numpy()), cs["down"])
    assert orc.rel_l2(d.float().cpu().numpy(), want_d) < TOL_GEMM


def _dn_layer(gpu, orc, H, T, Z, I, gs, zeros=False):
    cs = {}
    for i, (name, k, n) in enumerate((("in_qkv", H, T), ("in_z", H, Z), ("out", Z, H), ("gate", H, I),
                                       ("up", H, I), ("down", I, H))):
        cs[name] = orc.gptq_case(320 + i, k, n, gs, zeros=zeros)
    ws = {n: up(gpu, c) for n, c in cs.items()}
    return cs, sta.DeltaNetLinears(ws["in_qkv"], ws["in_z"], ws["out"], ws["gate"], ws["up"], ws["down"])


@pytest.mark.parametrize("Mr", [1, 5])
def test_deltanet_linears_decode(gpu, orc, Mr):
    """A DeltaNet layer's projections for 1-32 tokens (f32): in_proj_qkv |
    in_proj_z as one linear, out_proj on silu(z) * core (the reference's
    fused_silu_gptq_down, src/model.rs:786-791; at several tokens z is
    copied out of the strided qkv|z rows), the MLP, each against f64."""
    H, T, Z, I, gs = 256, 384, 128, 512, 128
    cs, layer = _dn_layer(gpu, orc, H, T, Z, I, gs, zeros=True)
    rng = np.random.default_rng(40 + Mr)
    x = rng.standard_normal((Mr, H)).astype(np.float32)
    core = rng.standard_normal((Mr, Z)).astype(np.float32)
    qkvz = torch.empty(Mr, T + Z, device="cuda")
    o, h, d = torch.empty(Mr, H, device="cuda"), torch.empty(Mr, I, device="cuda"), torch.empty(Mr, H, device="cuda")
    layer.decode(gpu, torch.from_numpy(x).cuda(), torch.from_numpy(core).cuda(), qkvz, o, h, d)
    torch.cuda.synchronize()
    y = qkvz.cpu().numpy()
    assert orc.rel_l2(y[:, :T], ref(orc, x, cs["in_qkv"])) < TOL_DECODE
    assert orc.rel_l2(y[:, T:], ref(orc, x, cs["in_z"])) < TOL_DECODE
    # out_proj on the z this call produced
    assert orc.rel_l2(o.cpu().numpy(), ref(orc, orc.silu_gate_f64(y[:, T:], core), cs["out"])) < TOL_DECODE
    want_h = orc.silu_gate_f64(ref(orc, x, cs["gate"]), ref(orc, x, cs["up"]))
    assert orc.rel_l2(h.cpu().numpy(), want_h) < TOL_DECODE
    assert orc.rel_l2(d.cpu().numpy(), ref(orc, h.cpu().numpy(), cs["down"])) < TOL_DECODE


def test_deltanet_linears_prefill(gpu, orc):
    """The same for a 40-token block (f16) through the GEMM: out_proj is
    st_gptq_i4_silu_gemm on z and the core's output."""
    H, T, Z, I, gs, Mr = 256, 384, 128, 512, 128, 40
    cs, layer = _dn_layer(gpu, orc, H, T, Z, I, gs)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((Mr, H)).astype(np.float16)
    core = rng.standard_normal((Mr, Z)).astype(np.float16)
    f16 = dict(device="cuda", dtype=torch.float16)
    qkvz, o = torch.empty(Mr, T + Z, **f16), torch.empty(Mr, H, **f16)
    g, u, d = torch.empty(Mr, I, **f16), torch.empty(Mr, I, **f16), torch.empty(Mr, H, **f16)
    layer.prefill(gpu, torch.from_numpy(x).cuda(), torch.from_numpy(core).cuda(), qkvz, o, g, u, d)
    torch.cuda.synchronize()
    y = qkvz.float().cpu().numpy()
    assert orc.rel_l2(y[:, :T], ref(orc, x, cs["in_qkv"])) < TOL_GEMM
    assert orc.rel_l2(y[:, T:], ref(orc, x, cs["in_z"])) < TOL_GEMM
    want_o = ref(orc, orc.silu_gate_f64(qkvz[:, T:].cpu().numpy(), core), cs["out"])
    assert orc.rel_l2(o.float().cpu().numpy(), want_o) < TOL_GEMM
    want_d = ref(orc, orc.silu_gate_f64(g.cpu().numpy(), u.cpu().numpy()), cs["down"])
    assert orc.rel_l2(d.float().cpu().numpy(), want_d) < TOL_GEMM


def test_decoder_linears_shape_checks(gpu, orc):
    cs, layer = _layer(gpu, orc, 256, 256, 128, 512, 128)
    x = torch.zeros(40, 256, device="cuda")
    with pytest.raises(ValueError):
        layer.decode(gpu, x, torch.zeros(40, 256, device="cuda"), None, None, None, None)
    w = {n: up(gpu, c) for n, c in cs.items()}
    with pytest.raises(ValueError):
        sta.DecoderLinears(w["q"], w["k"], w["v"], w["o"], w["gate"], w["up"], w["o"])


def test_decoder_linears_from_checkpoint_names(gpu, orc):
    """DecoderLinears.from_linears picks a layer's projections by the
    reference loader's tensor names and computes what the direct
    construction computes, bit for bit; a missing projection is a KeyError."""
    H, Q, KV, I, gs, Mr = 256, 256, 128, 512, 128, 2
    cs = {n: orc.gptq_case(400 + i, k, m, gs) for i, (n, k, m) in enumerate(
        (("q", H, Q), ("k", H, KV), ("v", H, KV), ("o", Q, H), ("gate", H, I), ("up", H, I), ("down", I, H)))}
    ws = {n: up(gpu, c) for n, c in cs.items()}
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    linears = {f"model.layers.3.{names[n]}": w for n, w in ws.items()}
    a = sta.DecoderLinears.from_linears(linears, 3)
    b = sta.DecoderLinears(ws["q"], ws["k"], ws["v"], ws["o"], ws["gate"], ws["up"], ws["down"])
    x = torch.randn(Mr, H, device="cuda")
    attn = torch.randn(Mr, Q, device="cuda")
    outs = []
    for layer in (a, b):
        bufs = [torch.empty(Mr, n, device="cuda") for n in (Q + 2 * KV, H, I, H)]
        layer.decode(gpu, x, attn, *bufs)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy() for t in bufs])
    for p_, q_ in zip(*outs):
        assert np.array_equal(p_, q_)
    del linears["model.layers.3.mlp.up_proj"]
    with pytest.raises(KeyError):
        sta.DecoderLinears.from_linears(linears, 3)


def test_gemm_argument_errors(gpu, orc):
    """The prefill entry points reject bad arguments with a status (the
    reference panics there) and launch nothing: NULL operands, a group size
    outside {64, 128, 256}, K not a multiple of 128, N not a multiple of 8,
    an output dtype other than f32/f16, misaligned A."""
    from shady_thinker_amd import _lib as L
    from shady_thinker_amd.gpu import ptr as p
    INVALID, SHAPE, ALIGN = 1, 2, 3  # st_status (include/shady_hip.h)
    K, N, Mr = 256, 64, 8
    c = orc.gptq_case(62, K, N, 128)
    w = up(gpu, c)
    a = torch.randn(Mr, K, device="cuda").half()
    u = torch.randn(Mr, K, device="cuda").half()
    y = torch.full((Mr, N), 3.0, device="cuda")
    gpu.sync_stream()

    def gemm(a_, k=K, n=N, gs=128, dt=L.ST_F32):
        L.call("st_gptq_i4_gemm", gpu.handle, a_, p(w.qweight), p(w.scales), None, None, p(y), dt, Mr, k, n, gs,
               w.flags)

    def silu(g_, u_, k=K, n=N, gs=128, dt=L.ST_F32):
        L.call("st_gptq_i4_silu_gemm", gpu.handle, g_, u_, p(w.qweight), p(w.scales), None, None, p(y), dt, Mr, k,
               n, gs, w.flags)

    cases = [
        (lambda: gemm(None), INVALID),
        (lambda: gemm(p(a), gs=32), SHAPE),
        (lambda: gemm(p(a), k=200), SHAPE),
        (lambda: gemm(p(a), n=60), SHAPE),
        (lambda: gemm(p(a), dt=L.ST_BF16), INVALID),
        (lambda: gemm(p(a) + 2), ALIGN),
        (lambda: silu(p(a), None), INVALID),
        (lambda: silu(None, p(u)), INVALID),
        (lambda: silu(p(a), p(u), gs=512), SHAPE),
    ]
    for fn, code in cases:
        with pytest.raises(L.ShadyHipError) as ei:
            fn()
        assert ei.value.code == code, str(ei.value)
    torch.cuda.synchronize()
    assert bool((y == 3.0).all())  # nothing was written
