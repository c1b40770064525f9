"""GPU parity of the INT8 prefill GEMM st_int8_gemm (W8A16) against the CPU
oracle, through the C ABI.

The kernel forms every product int8 x f16 exactly in f32 on the f16 MFMA
(both operands are exact in f16) and applies the channel scale once per
output, so only the f32 sums round: it is checked against the f64 oracle far
below the GEMM bar (2e-3), bit for bit where the sums are exact integers, and
at configs[2]'s shape (K=5120, N=13824) at prefill M on a row/column sample.
"""
import numpy as np
import pytest
import torch

import shady_thinker_amd as sta
from shady_thinker_amd import model as M

pytestmark = pytest.mark.gpu

TOL = 2e-3  # rel-L2, prefill GEMM (north_star)
TIGHT = 1e-5  # f32 sums of exact products (observed ~1e-7)


def run(gpu, w, a_np, out_dtype=torch.float32):
    a = torch.from_numpy(np.ascontiguousarray(a_np, dtype=np.float16)).to(gpu.device)
    c = torch.empty(a.shape[0], w.N, dtype=out_dtype, device=gpu.device)
    M.int8_gemm(gpu, a, w.w, w.scale, c, w.K, w.N, w.flags)
    torch.cuda.synchronize()
    return c.float().cpu().numpy()


@pytest.mark.parametrize("tiled", [True, False])
@pytest.mark.parametrize("Mr,K,N", [
    (1, 128, 4),
    (33, 256, 260),
    (130, 1024, 1000),
    (257, 2048, 520),
    (40, 4096, 256),   # few tiles: K split across workgroups
    (600, 640, 2052),
])
def test_int8_gemm_matches_oracle(gpu, orc, tiled, Mr, K, N):
    c = orc.int8_case(30 + Mr, K, N, M=Mr)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"], tiled=tiled)
    y = run(gpu, w, c["x"])
    ref = orc.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)
    e = orc.rel_l2(y, ref)
    print(f"int8 gemm M={Mr} K={K} N={N} tiled={tiled}: rel-L2 {e:.3e}")
    assert e < TIGHT


@pytest.mark.parametrize("tiled", [True, False])
def test_int8_gemm_integer_exact(gpu, orc, tiled):
    """Integer activations and unit scales: every partial sum is an integer
    below 2^24, so C must equal the int64 product exactly. Pins the byte
    order, the k pairing of A and B and the row/column mapping."""
    Mr, K, N = 161, 1024, 388
    rng = np.random.default_rng(7)
    w = rng.integers(-127, 128, size=(N, K), dtype=np.int64).astype(np.int8)
    a = rng.integers(-8, 9, size=(Mr, K)).astype(np.float16)
    wt = sta.Int8Weight.upload(gpu, w, np.ones(N, np.float32), tiled=tiled)
    y = run(gpu, wt, a)
    ref = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.abs(ref).max() < 2 ** 24
    np.testing.assert_array_equal(y, ref.astype(np.float32))


@pytest.mark.parametrize("N", [776, 388])
def test_int8_gemm_f16_output_and_layouts_agree(gpu, orc, N):
    """f16 C equals the f32 C rounded, in both epilogues: rows staged through
    LDS as 16-byte chunks (N % 8 == 0) and per-element stores (N = 388)."""
    Mr, K = 300, 1536
    c = orc.int8_case(9, K, N, M=Mr)
    wt = sta.Int8Weight.upload(gpu, c["w"], c["scale"], tiled=True)
    wr = sta.Int8Weight.upload(gpu, c["w"], c["scale"], tiled=False)
    yt = run(gpu, wt, c["x"])
    yr = run(gpu, wr, c["x"])
    assert orc.rel_l2(yt, yr) < 1e-6
    h = run(gpu, wt, c["x"], torch.float16)
    np.testing.assert_array_equal(h, yt.astype(np.float16).astype(np.float32))


def test_int8_gemm_cfg2_prefill_full_size(gpu, orc):
    """configs[2]'s weight (K=5120, N=13824, int8 uniform -127..127, f32
    scales |N(0, 0.01)|) at prefill M=2048, f16 activations N(0, 1): the full
    C checked against the f64 oracle on 64 rows x 512 columns (first, last
    and strided), and the split-free whole against the row-major layout."""
    K, N, Mr = 5120, 13824, 2048
    c = orc.int8_case(2, K, N, M=Mr)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"], tiled=True)
    y = run(gpu, w, c["x"])
    assert np.isfinite(y).all()
    rows = np.unique(np.r_[0, Mr - 1, np.linspace(1, Mr - 2, 62).astype(int)])
    cols = np.unique(np.r_[0, N - 1, np.linspace(1, N - 2, 510).astype(int)])
    ref = orc.int8_matvec_f64(c["x"][rows], c["w"][cols], c["scale"][cols], K, len(cols))
    e = orc.rel_l2(y[np.ix_(rows, cols)], ref)
    print(f"int8 gemm configs[2] M={Mr}: rel-L2 {e:.3e} on {len(rows)}x{len(cols)}")
    assert e < TIGHT


def test_int8_linear_dispatches_gemm_above_32_tokens(gpu, orc):
    """linear() on an Int8Weight: 48 tokens of f32 x go to st_int8_gemm on
    x rounded to f16 (the matvec entry point stops at 32)."""
    Mr, K, N = 48, 1024, 512
    c = orc.int8_case(4, K, N, M=Mr, x_dtype=np.float32)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
    x = torch.from_numpy(c["x"]).to(gpu.device)
    y = torch.empty(Mr, N, device=gpu.device)
    M.linear(gpu, x, w, y)
    torch.cuda.synchronize()
    ref = orc.int8_matvec_f64(c["x"].astype(np.float16), c["w"], c["scale"], K, N)
    assert orc.rel_l2(y.cpu().numpy(), ref) < TIGHT


def test_int8_gemm_graph_replay(gpu, orc):
    """Captured once, replayed three times with eager work between: every
    replay equals the eager result bit for bit (split-K grid included)."""
    for Mr, K, N in ((40, 4096, 256), (260, 1024, 1032)):
        c = orc.int8_case(11, K, N, M=Mr)
        w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
        a = torch.from_numpy(c["x"]).to(gpu.device)
        eager = torch.empty(Mr, N, device=gpu.device)
        M.int8_gemm(gpu, a, w.w, w.scale, eager, K, N, w.flags)
        torch.cuda.synchronize()
        out = torch.empty_like(eager)
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            M.int8_gemm(gpu, a, w.w, w.scale, out, K, N, w.flags)  # warm on s
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                M.int8_gemm(gpu, a, w.w, w.scale, out, K, N, w.flags)
        for i in range(3):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            with torch.cuda.stream(s):
                graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"M={Mr} replay {i}"
            M.int8_gemm(gpu, a, w.w, w.scale, eager, K, N, w.flags)  # eager work between
            torch.cuda.synchronize()


def test_int8_gemm_split_k_matches_unsplit(gpu, orc, tune):
    """Few tiles split K across workgroups (scaled f32 partials, added in a
    fixed order): the oracle's result either way, and the same as one
    workgroup per tile up to summation order."""
    Mr, K, N = 64, 4096, 264
    c = orc.int8_case(61, K, N, M=Mr)
    w = sta.Int8Weight.upload(gpu, c["w"], c["scale"])
    y_split = run(gpu, w, c["x"])
    tune(GEMM_NO_SPLIT=1)
    y_one = run(gpu, w, c["x"])
    ref = orc.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)
    assert orc.rel_l2(y_split, ref) < TIGHT and orc.rel_l2(y_one, ref) < TIGHT
    assert orc.rel_l2(y_split, y_one) < 1e-6
