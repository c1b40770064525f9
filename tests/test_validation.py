"""Host-side argument checks (CPU, no GPU): the C ABI takes bare pointers,
so the Python helpers and the upload path refuse a wrong dtype, a
non-contiguous tensor or a buffer shorter than the shape needs before any
device call (otherwise a kernel would read or write past an allocation).
Tensors here are CPU tensors and the context is a stand-in: a check that
let a call through would reach the C ABI with a NULL context and fail with
ShadyHipError instead of the TypeError / ValueError asserted."""
import os

import numpy as np
import pytest
import torch

from shady_thinker_amd import model as M
from shady_thinker_amd._lib import ST_FLAG_TILED, ShadyHipError, lib
from shady_thinker_amd.loader import read_gptq_checkpoint
from shady_thinker_amd.weights import GptqWeight, check_gptq_tensors


class NoGpu:
    handle = None

    def sync_stream(self):
        pass


K, N, GS = 256, 64, 128


def gptq(tiled=False):
    words = lib().st_gptq_i4_tiled_words(K, N, GS) if tiled else K // 8 * N
    return (torch.zeros(words, dtype=torch.int32), torch.zeros(K // GS, N, dtype=torch.float16),
            torch.zeros(K // GS, N // 8, dtype=torch.int32), torch.zeros(K, dtype=torch.int32))


def mv(x=None, qw=None, sc=None, y=None, qz=None, perm=None, flags=0, m=1):
    q0, s0, _, _ = gptq(bool(flags & ST_FLAG_TILED))
    M.gptq_matvec(NoGpu(), "t", torch.zeros(m, K) if x is None else x, q0 if qw is None else qw,
                  s0 if sc is None else sc, torch.zeros(m, N) if y is None else y, K, N, GS, qz, perm, flags)


def test_valid_arguments_reach_the_c_abi():
    with pytest.raises(ShadyHipError):  # NULL context: the checks let it through
        mv()
    q0, s0, z0, p0 = gptq(True)
    with pytest.raises(ShadyHipError):
        mv(qw=q0, qz=z0, perm=p0, flags=ST_FLAG_TILED)


@pytest.mark.parametrize("kw,exc", [
    (dict(y=torch.zeros(1, N, dtype=torch.float16)), TypeError),     # f16 output of an f32 kernel
    (dict(y=torch.zeros(1, N - 1)), ValueError),                     # output too short
    (dict(y=torch.zeros(N, 2)[:, 0]), ValueError),                   # non-contiguous output
    (dict(sc=torch.zeros(K // GS, N)), TypeError),                   # f32 scales
    (dict(sc=torch.zeros(K // GS, N - 8, dtype=torch.float16)), ValueError),
    (dict(qw=torch.zeros(K // 8 * N - 1, dtype=torch.int32)), ValueError),
    (dict(qw=torch.zeros(K // 8 * N, dtype=torch.int16)), TypeError),
    (dict(qz=torch.zeros(K // GS, N // 8 - 1, dtype=torch.int32)), ValueError),
    (dict(perm=torch.zeros(K, dtype=torch.int64)), TypeError),
    (dict(perm=torch.zeros(K - 1, dtype=torch.int32)), ValueError),
    (dict(x=torch.zeros(1, K, dtype=torch.bfloat16)), TypeError),
    (dict(x=torch.zeros(K, 2)[:, 0].reshape(1, K)), ValueError),   # non-contiguous input
    (dict(x=torch.zeros(K + 8)), ValueError),                        # not a whole number of rows
    (dict(x=torch.zeros(0, K)), ValueError),                         # no rows
])
def test_matvec_rejects(kw, exc):
    with pytest.raises(exc):
        mv(**kw)


def test_tiled_qweight_size_is_checked():
    Kt, Nt = 256, 72
    words = lib().st_gptq_i4_tiled_words(Kt, Nt, GS)
    assert words > Kt // 8 * Nt
    with pytest.raises(ValueError):
        M.gptq_matvec(NoGpu(), "t", torch.zeros(1, Kt), torch.zeros(Kt // 8 * Nt, dtype=torch.int32),
                      torch.zeros(Kt // GS, Nt, dtype=torch.float16), torch.zeros(1, Nt), Kt, Nt, GS,
                      flags=ST_FLAG_TILED)


def test_gemm_needs_f16_a_and_linear_converts():
    q0, s0, _, _ = gptq()
    a32 = torch.zeros(48, K)
    with pytest.raises(TypeError):
        M.gptq_gemm(NoGpu(), a32, q0, s0, torch.zeros(48, N), K, N, GS)
    with pytest.raises(TypeError):
        M.fused_silu_gptq_gemm(NoGpu(), a32, a32, q0, s0, torch.zeros(48, N), K, N, GS)
    with pytest.raises(TypeError):  # C is f32 or f16
        M.gptq_gemm(NoGpu(), a32.half(), q0, s0, torch.zeros(48, N, dtype=torch.bfloat16), K, N, GS)
    w = GptqWeight(q0, s0, None, None, K, N, GS, 0)
    with pytest.raises(ShadyHipError):  # f32 x of 48 tokens: rounded to f16, then the GEMM call
        M.linear(NoGpu(), a32, w, torch.zeros(48, N))


def test_int8_and_bf16_reject_short_buffers():
    x, y = torch.zeros(1, K, dtype=torch.float16), torch.zeros(1, N)
    with pytest.raises(ValueError):
        M.int8_matvec(NoGpu(), x, torch.zeros(K * N - 1, dtype=torch.int8), torch.zeros(N), y, K, N)
    with pytest.raises(TypeError):
        M.int8_matvec(NoGpu(), x, torch.zeros(K * N, dtype=torch.int8), torch.zeros(N, dtype=torch.float16), y, K, N)
    Kt, Nt = 256, 72  # the tiled layout pads N to 16 rows: K * N bytes are too few
    assert lib().st_int8_tiled_bytes(Kt, Nt) > Kt * Nt
    with pytest.raises(ValueError):
        M.int8_matvec(NoGpu(), torch.zeros(1, Kt, dtype=torch.float16), torch.zeros(Kt * Nt, dtype=torch.int8),
                      torch.zeros(Nt), torch.zeros(1, Nt), Kt, Nt, ST_FLAG_TILED)
    with pytest.raises(ValueError):
        M.bf16_matvec(NoGpu(), x, torch.zeros(N * K - 1, dtype=torch.int16), y, K, N)


def test_int8_gemm_checks_and_linear_routes_it():
    from shady_thinker_amd.weights import Int8Weight

    w8, sc = torch.zeros(K * N, dtype=torch.int8), torch.zeros(N)
    a16, c = torch.zeros(48, K, dtype=torch.float16), torch.zeros(48, N)
    with pytest.raises(ShadyHipError):  # valid: reaches the C ABI (NULL context)
        M.int8_gemm(NoGpu(), a16, w8, sc, c, K, N)
    with pytest.raises(TypeError):  # f32 activations
        M.int8_gemm(NoGpu(), a16.float(), w8, sc, c, K, N)
    with pytest.raises(TypeError):  # C is f32 or f16
        M.int8_gemm(NoGpu(), a16, w8, sc, c.to(torch.bfloat16), K, N)
    with pytest.raises(ValueError):  # C too short
        M.int8_gemm(NoGpu(), a16, w8, sc, torch.zeros(47, N), K, N)
    with pytest.raises(ValueError):  # short weight
        M.int8_gemm(NoGpu(), a16, w8[:-1], sc, c, K, N)
    with pytest.raises(TypeError):  # f16 channel scales
        M.int8_gemm(NoGpu(), a16, w8, sc.half(), c, K, N)
    Kt, Nt = 256, 72  # tiled: K * N bytes are too few
    with pytest.raises(ValueError):
        M.int8_gemm(NoGpu(), a16[:, :Kt], torch.zeros(Kt * Nt, dtype=torch.int8), torch.zeros(Nt),
                    torch.zeros(48, Nt), Kt, Nt, ST_FLAG_TILED)
    w = Int8Weight(w8, sc, K, N, 0)
    with pytest.raises(ShadyHipError):  # 48 tokens of f32 x: rounded to f16, then the GEMM call
        M.linear(NoGpu(), a16.float(), w, c)


def test_upload_tensor_checks():
    qw = np.zeros((K // 8, N), np.int32)
    sc = np.zeros((K // GS, N), np.float16)
    check_gptq_tensors(qw, sc, GS, np.zeros((K // GS, N // 8), np.int32), np.arange(K) // GS)
    with pytest.raises(ValueError):  # f32 scales are refused, not reinterpreted
        check_gptq_tensors(qw, sc.astype(np.float32), GS)
    with pytest.raises(ValueError):
        check_gptq_tensors(qw, sc[:, :-8], GS)
    with pytest.raises(ValueError):
        check_gptq_tensors(qw, sc, GS, np.zeros((K // GS, N // 8 + 1), np.int32))
    with pytest.raises(ValueError):
        check_gptq_tensors(qw, sc, GS, None, np.arange(K - 1) // GS)
    with pytest.raises(ValueError):
        check_gptq_tensors(qw.astype(np.int64), sc, GS)
    with pytest.raises(ValueError):
        check_gptq_tensors(qw, sc, 96)


def test_loader_refuses_bf16_scales(orc, tmp_path):
    from safetensors.torch import save_file

    d = str(tmp_path)
    c = orc.gptq_case(50, K, N, GS)
    save_file({"model.layers.0.self_attn.q_proj.qweight": torch.from_numpy(c["qweight"].view(np.int32)),
               "model.layers.0.self_attn.q_proj.scales": torch.zeros(K // GS, N, dtype=torch.bfloat16)},
              os.path.join(d, "model.safetensors"))
    with pytest.raises(ValueError, match="bfloat16"):
        read_gptq_checkpoint(d)
    save_file({"model.layers.0.self_attn.q_proj.qweight": torch.from_numpy(c["qweight"].view(np.int32)),
               "model.layers.0.self_attn.q_proj.scales": torch.from_numpy(c["scales"].view(np.float16)),
               "model.layers.0.self_attn.q_proj.qzeros": torch.zeros(K // GS, N // 8 - 1, dtype=torch.int32)},
              os.path.join(d, "model.safetensors"))
    with pytest.raises(ValueError, match="qzeros"):
        read_gptq_checkpoint(d)
