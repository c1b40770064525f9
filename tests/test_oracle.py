"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own code path: numpy / torch
library conversions, exhaustive enumeration, closed forms (one-hot inputs,
integer-exact cases) and float64 matmuls. The reference ships no golden
vectors for this path (its tests only assert on generated text,
tests/integration/jit_lora_test.rs:19-60), so these are the pins.
"""
import os

import numpy as np
import pytest
import torch

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _xorshift_first(seed, n):
    # src/lora.rs:80-92 definition, written out for the first draws.
    m = (1 << 64) - 1
    s = seed ^ 0x5DEECE66D
    out = []
    for _ in range(n):
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        out.append(s)
    return out


def test_rng_matches_xorshift_definition(orc):
    for seed in (0, 1, 12345, 2**63 + 7):
        assert list(orc.rng_draws(seed, 5)) == _xorshift_first(seed, 5)


def test_rng_normal_moments(orc):
    z = orc.normal_f32(3, 200_000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01


def test_nibble_and_int8_generators_cover_range(orc):
    w = orc.nibbles(1, 20_000)
    nib = np.stack([(w >> (4 * j)) & 0xF for j in range(8)])
    counts = np.bincount(nib.ravel(), minlength=16)
    assert counts.min() > 0.9 * counts.mean()
    i8 = orc.int8(2, 100_000)
    assert i8.min() == -127 and i8.max() == 127
    p = orc.perm(4, 1000)
    assert np.array_equal(np.sort(p), np.arange(1000))


def test_f16_to_f32_exhaustive(orc):
    lib = orc.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(0)
    pats = rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32)
    vals = pats.view(np.float32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, 2**-24, 2**-25, 2**-25 * 1.0001, 3 * 2**-26,
                     6.1e-5, 5.96e-8, np.inf, -np.inf], np.float32)
    vals = np.concatenate([vals, edge, rng.normal(0, 0.02, 50_000).astype(np.float32)])
    lib = orc.lib()
    got = np.array([lib.orc_f32_to_f16(float(v)) for v in vals], np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    nan = np.isnan(vals)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


def test_f32_to_bf16_matches_torch(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.normal(0, 1, 20_000), rng.normal(0, 1e-30, 1000), [0.0, -0.0, 3.0e38, np.inf]])
    vals = vals.astype(np.float32)
    lib = orc.lib()
    got = np.array([lib.orc_f32_to_bf16(float(v)) for v in vals], np.uint16)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_dequant_kat_exhaustive(orc):
    """All 16 q x 16 z x 65,536 f16 scale patterns: (f32(q) - f32(z)) * f32(s)
    bit-equal to numpy float32 and to the exact float64 product."""
    K, gs, N = 256, 16, 65536
    # row k holds q = k % 16 in every column; group g = k // 16 has zero g.
    q = np.arange(K) % 16
    words = np.zeros((K // 8, N), np.uint32)
    for j in range(8):
        words |= (q[j::8].astype(np.uint32)[:, None] << np.uint32(4 * j))
    scales = np.tile(np.arange(65536, dtype=np.uint16), (K // gs, 1))
    zrow = np.zeros(N // 8, np.uint32)
    qz = np.stack([zrow | np.uint32(sum(g << (4 * j) for j in range(8))) for g in range(16)])
    out = orc.gptq_dequant_f32(words, scales.view(np.float16), K, N, gs, qzeros=qz)
    s32 = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    ref32 = (q.astype(np.float32)[:, None] - (np.arange(K) // gs).astype(np.float32)[:, None]) * s32[None, :]
    ref64 = (q.astype(np.float64)[:, None] - (np.arange(K) // gs)[:, None]) * s32.astype(np.float64)[None, :]
    nan = np.isnan(ref32)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), ref32[~nan].view(np.uint32))
    fin = np.isfinite(ref64)
    assert np.array_equal(out[fin].astype(np.float64), ref64[fin])


def test_dequant_scalar_matches_table(orc):
    for qv, zv, sb in [(0, 8, 0x3C00), (15, 8, 0x2148), (7, 0, 0xBC00), (3, 3, 0x7BFF)]:
        expect = np.float32(qv - zv) * np.uint16(sb).view(np.float16).astype(np.float32)
        assert orc.dequant_i4(qv, zv, sb) == expect


def test_dequant_layout_nibble_positions(orc):
    """One nonzero nibble at a time lands at out[8 * pr + j, n] (the [K, N]
    transposition of src/weights.rs:295-311)."""
    K, N, gs = 64, 16, 32
    sc = np.full((K // gs, N), 1.0, np.float16)
    for pr, j, n in [(0, 0, 0), (3, 7, 5), (7, 4, 15), (5, 1, 9)]:
        qw = np.full((K // 8, N), 0x88888888, np.uint32)
        qw[pr, n] = (qw[pr, n] & ~np.uint32(0xF << (4 * j))) | np.uint32(0xF << (4 * j))
        out = orc.gptq_dequant_f32(qw, sc, K, N, gs)
        expect = np.zeros((K, N), np.float32)
        expect[8 * pr + j, n] = 7.0
        assert np.array_equal(out, expect)


def test_dequant_bf16_is_rne_of_f32(orc):
    c = orc.gptq_case(7, 256, 64)
    f32 = orc.gptq_dequant_f32(c["qweight"], c["scales"], 256, 64, 128)
    bf = orc.gptq_dequant_bf16(c["qweight"], c["scales"], 256, 64, 128)
    ref = torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf, ref)


@pytest.mark.parametrize("K,N,gs", [(256, 64, 128), (2048, 256, 128), (512, 40, 64)])
def test_f64_matvec_equals_numpy_matmul(orc, K, N, gs):
    for zeros, act in [(False, False), (True, False), (True, True)]:
        c = orc.gptq_case(11, K, N, gs, zeros=zeros, act_order=act, M=3)
        W = orc.gptq_dequant_f32(c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
        ref = c["x"].astype(np.float64) @ W.astype(np.float64)
        got = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
        assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_act_order_scales_follow_g_idx(orc):
    """A permuted g_idx must pick scales[g_idx[k]]: checked against dequant
    with rows/scales rearranged by hand."""
    K, N, gs = 256, 16, 64
    c = orc.gptq_case(5, K, N, gs, act_order=True)
    W = orc.gptq_dequant_f32(c["qweight"], c["scales"], K, N, gs, g_idx=c["g_idx"])
    sc = c["scales"].astype(np.float32)
    for k in (0, 17, 100, 255):
        q = (c["qweight"][k // 8] >> np.uint32(4 * (k % 8))) & np.uint32(0xF)
        assert np.array_equal(W[k], (q.astype(np.float32) - 8.0) * sc[c["g_idx"][k]])


def test_one_hot_matvec_returns_dequant_row(orc):
    K, N, gs = 512, 64, 128
    c = orc.gptq_case(2, K, N, gs, zeros=True)
    W = orc.gptq_dequant_f32(c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"])
    for k in (0, 129, 511):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        y = orc.gptq_matvec_f64(x, c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"])
        assert np.array_equal(y, W[k].astype(np.float64))
        y32 = orc.gptq_matvec_wgsl(x, c["qweight"], c["scales"], K, N, gs)
        Wsym = orc.gptq_dequant_f32(c["qweight"], c["scales"], K, N, gs)
        assert np.array_equal(y32, Wsym[k])


def test_symmetric_zeros_equal_reference_mode(orc):
    """qzeros all 8 (raw) or all 7 with the +1 convention == the reference's
    hard-coded zero point 8 (gptq_matvec.wgsl:51)."""
    K, N, gs = 256, 64, 128
    c = orc.gptq_case(3, K, N, gs)
    base = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs)
    z8 = np.full((K // gs, N // 8), 0x88888888, np.uint32)
    z7 = np.full((K // gs, N // 8), 0x77777777, np.uint32)
    assert np.array_equal(orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=z8), base)
    assert np.array_equal(
        orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, qzeros=z7, zero_offset=1), base)
    ident = (np.arange(K) // gs).astype(np.int32)
    assert np.array_equal(orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, gs, g_idx=ident), base)


def test_wgsl_order_integer_exact(orc):
    """Scales 1.0 and small integer x: every WGSL-order f32 sum is exact, so
    1t, 4t, with and without FMA all equal the f64 result bit for bit."""
    K, N, gs = 1024, 64, 128
    c = orc.gptq_case(9, K, N, gs)
    sc = np.ones_like(c["scales"])
    x = np.round(c["x"] * 3).astype(np.float32)
    ref = orc.gptq_matvec_f64(x, c["qweight"], sc, K, N, gs).astype(np.float32)
    for v in (0, 1):
        for ct in (0, 1):
            assert np.array_equal(orc.gptq_matvec_wgsl(x, c["qweight"], sc, K, N, gs, v, ct), ref)


def test_wgsl_order_close_to_f64(orc):
    K = N = 2048
    c = orc.gptq_case(0, K, N, 128)
    ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, 128)
    for v in (0, 1):
        for ct in (0, 1):
            y = orc.gptq_matvec_wgsl(c["x"], c["qweight"], c["scales"], K, N, 128, v, ct)
            assert orc.rel_l2(y, ref) < 5e-6


def test_silu_paths(orc):
    K, N, gs = 512, 64, 128
    c = orc.gptq_case(4, K, N, gs)
    a = orc.normal_f32(100, K) * 3
    b = orc.normal_f32(101, K)
    xs = orc.silu_mul_f64(a, b)
    # closed form of silu on a = 0 and large |a|
    assert np.array_equal(orc.silu_mul_f64(np.zeros(4, np.float32), np.ones(4, np.float32)), np.zeros(4))
    big = orc.silu_mul_f64(np.array([40.0], np.float32), np.array([2.0], np.float32))
    assert abs(big[0] - 80.0) < 1e-12
    np.testing.assert_allclose(xs, a.astype(np.float64) / (1 + np.exp(-a.astype(np.float64))) * b, rtol=1e-15)
    ref = orc.gptq_matvec_f64(xs, c["qweight"], c["scales"], K, N, gs)
    for v in (0, 1):
        y = orc.fused_silu_gptq_wgsl(a, b, c["qweight"], c["scales"], K, N, gs, v, 1)
        assert orc.rel_l2(y, ref) < 1e-5


def test_gate_up_paths(orc):
    K, N, gs = 512, 64, 128
    cg = orc.gptq_case(6, K, N, gs)
    cu = orc.gptq_case(8, K, N, gs)
    x = cg["x"]
    g = orc.gptq_matvec_f64(x, cg["qweight"], cg["scales"], K, N, gs)
    u = orc.gptq_matvec_f64(x, cu["qweight"], cu["scales"], K, N, gs)
    ref = orc.silu_gate_f64(g, u)
    np.testing.assert_allclose(ref, g / (1 + np.exp(-g)) * u, rtol=1e-14)
    for v in (0, 1):
        y = orc.gate_up_silu_wgsl(x, cg["qweight"], cg["scales"], cu["qweight"], cu["scales"], K, N, gs, v, 1)
        assert orc.rel_l2(y, ref) < 1e-5


def test_int8_f64_equals_numpy(orc):
    c = orc.int8_case(1, 512, 96, M=4)
    ref = (c["x"].astype(np.float64) @ c["w"].T.astype(np.float64)) * c["scale"].astype(np.float64)
    got = orc.int8_matvec_f64(c["x"], c["w"], c["scale"], 512, 96)
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=1e-13)


def test_golden_fixtures_reproduce(orc):
    """The committed fixtures (tests/golden/make_golden.py) still match the
    oracle: a regression pin on generator + oracle together."""
    files = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))
    assert files, "no golden fixtures"
    for f in files:
        d = np.load(os.path.join(GOLDEN, f))
        kind = str(d["kind"])
        if kind == "int8":
            y = orc.int8_matvec_f64(d["x"], d["w"], d["scale"], int(d["K"]), int(d["N"]))
        else:
            x = d["x"]
            if kind == "silu":
                x = orc.silu_mul_f64(d["a"], d["b"])
            y = orc.gptq_matvec_f64(x, d["qweight"], d["scales"], int(d["K"]), int(d["N"]), int(d["gs"]),
                                    qzeros=d["qzeros"] if d["qzeros"].size else None,
                                    g_idx=d["g_idx"] if d["g_idx"].size else None)
        assert np.array_equal(y, d["y"]), f


def test_bf16_matvec_oracle_pins(orc):
    """bf16 matvec oracle: f64 truth equals numpy float64 on the exact f32
    values of the bf16 bits; the WGSL-order f32 path equals it bit for bit on
    an integer-exact case (small integer weights and x) and stays within
    1e-6 rel-L2 on random data; bf16 generation is RNE (matches torch)."""
    import torch

    K, N = 136, 40
    c = orc.bf16_case(5, K, N, 2)
    Wf = (c["w"].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    ref = c["x"].astype(np.float64) @ Wf.T
    assert np.allclose(orc.bf16_matvec_f64(c["x"], c["w"], K, N), ref, rtol=1e-12, atol=1e-12)
    for contract in (0, 1):
        wg = orc.bf16_matvec_wgsl(c["x"][0], c["w"], K, N, contract)
        assert orc.rel_l2(wg, ref[0]) < 1e-6
    rng = np.random.default_rng(1)
    wi = rng.integers(-8, 9, size=(N, K)).astype(np.float32)
    xi = rng.integers(-4, 5, size=K).astype(np.float32)
    wbits = orc._bf16_bits(wi)
    exact = orc.bf16_matvec_f64(xi, wbits, K, N)
    assert np.array_equal(orc.bf16_matvec_wgsl(xi, wbits, K, N).astype(np.float64), exact)
    v = rng.standard_normal(4096).astype(np.float32)
    assert np.array_equal(orc._bf16_bits(v), torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
