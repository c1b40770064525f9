"""GPU parity of the bf16 matvec (st_bf16_matvec, the lm_head / tied
embedding projection of src/shaders/bf16_matvec.wgsl) through the C ABI.

Bar: f32-accumulate matvec, rel-L2 <= 1e-4 against the f64 oracle and the
WGSL-order f32 restatement (north_star); one-hot x returns a weight column
exactly (single bf16 * 1.0 products, exact in f32).
"""
import numpy as np
import pytest
import torch

import shady_thinker_amd as sta
from shady_thinker_amd import model as M

pytestmark = pytest.mark.gpu

TOL = 1e-4


def run(gpu, w_bits, x, xdtype=torch.float32):
    w = torch.from_numpy(np.ascontiguousarray(w_bits).view(np.int16)).to(gpu.device)
    xt = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu.device).to(xdtype)
    y = torch.empty(xt.shape[0], w.shape[0], device=gpu.device)
    M.bf16_matvec(gpu, xt, w, y, w.shape[1], w.shape[0])
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("K,N,Mr", [(64, 8, 1), (72, 13, 1), (2560, 1000, 1), (2560, 1000, 2), (1032, 777, 4),
                                    (4096, 4099, 3), (2560, 600, 8), (520, 33, 5)])
def test_bf16_matvec_matches_oracle(gpu, orc, K, N, Mr):
    c = orc.bf16_case(20 + K + Mr, K, N, Mr)
    y = run(gpu, c["w"], c["x"])
    ref = orc.bf16_matvec_f64(c["x"], c["w"], K, N)
    e = orc.rel_l2(y, ref)
    wg = orc.bf16_matvec_wgsl(c["x"][0], c["w"], K, N)
    ew = orc.rel_l2(y[0], wg)
    print(f"bf16 K={K} N={N} M={Mr}: rel-L2 vs f64 {e:.3e}, vs WGSL order {ew:.3e}")
    assert e < TOL and ew < TOL
    assert e < 1e-6


def test_bf16_matvec_f16_x(gpu, orc):
    K, N = 2560, 513
    c = orc.bf16_case(7, K, N, 4)
    x16 = c["x"].astype(np.float16)
    y = run(gpu, c["w"], x16.astype(np.float32), torch.float16)
    ref = orc.bf16_matvec_f64(x16, c["w"], K, N)
    assert orc.rel_l2(y, ref) < 1e-6


def test_bf16_one_hot_returns_columns_exactly(gpu, orc):
    K, N = 200, 77
    c = orc.bf16_case(3, K, N)
    W = (c["w"].astype(np.uint32) << 16).view(np.float32)  # [N, K] exact f32 values
    ks = [0, 1, 7, 8, 63, 64, 127, 199]
    x = np.zeros((len(ks[:4]), K), np.float32)
    for chunk in (ks[:4], ks[4:]):
        x[:] = 0
        for i, k in enumerate(chunk):
            x[i, k] = 1.0
        y = run(gpu, c["w"], x)
        for i, k in enumerate(chunk):
            assert np.array_equal(y[i], W[:, k]), k


def test_bf16_lm_head_full_size_vs_torch(gpu):
    """configs[4] lm_head: vocab 151936 x hidden 2560, batch 1 and 4, against
    a float64 torch matmul of the same bf16 values."""
    K, N = 2560, 151936
    g = torch.Generator(device=gpu.device)
    g.manual_seed(11)
    w = (torch.randn(N, K, generator=g, device=gpu.device) * 0.02).to(torch.bfloat16)
    for Mr in (1, 4):
        x = torch.randn(Mr, K, generator=g, device=gpu.device)
        y = torch.empty(Mr, N, device=gpu.device)
        M.bf16_matvec(gpu, x, w.view(torch.int16), y, K, N)
        ref = x.double() @ w.double().t()
        torch.cuda.synchronize()
        e = (torch.linalg.vector_norm((y.double() - ref)) / torch.linalg.vector_norm(ref)).item()
        print(f"lm_head M={Mr}: rel-L2 {e:.3e}")
        assert e < TOL and e < 1e-6


def test_bf16_errors(gpu):
    w = torch.zeros(8, 64, dtype=torch.int16, device=gpu.device)
    x = torch.zeros(9, 64, device=gpu.device)
    y = torch.empty(9, 8, device=gpu.device)
    with pytest.raises(sta.ShadyHipError):
        M.bf16_matvec(gpu, x, w, y, 64, 8)  # M = 9
    w2 = torch.zeros(8, 60, dtype=torch.int16, device=gpu.device)
    with pytest.raises(sta.ShadyHipError):
        M.bf16_matvec(gpu, x[:1, :60].contiguous(), w2, y[:1], 60, 8)  # K % 8
