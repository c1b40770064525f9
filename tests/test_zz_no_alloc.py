"""st_gptq_i4_matvec_noalloc (no reference counterpart: the decode matvec for
callers that cannot allocate, its workspace in the library's fixed per-GPU
scratch) against st_gptq_i4_matvec, through the C ABI: two calls in a row on
the shared scratch, the second smaller, each equal to the existing entry
point bit for bit (same kernels, same split decisions) and within the
north_star bar (rel-L2 1e-4) of the f64 oracle; and a call beyond the
scratch fails with a status and writes nothing."""
import numpy as np
import pytest
import torch

import shady_thinker_amd as sta
from shady_thinker_amd._lib import ST_ERR_WORKSPACE, ST_F32, call, lib

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _mv(gpu, fn, x, w, y):
    gpu.sync_stream()
    call(fn, gpu.handle, x.data_ptr(), ST_F32, w.qweight.data_ptr(), w.scales.data_ptr(),
         None if w.qzeros is None else w.qzeros.data_ptr(), None if w.perm is None else w.perm.data_ptr(),
         y.data_ptr(), x.shape[0], w.K, w.N, w.group_size, w.flags)


@pytest.mark.parametrize("first,second", [
    # (tokens, K, N, zeros): 16 tokens on 384 tiles take the f16-MFMA kernel;
    # 5 tokens on 160 tiles take the limb kernels with K split across
    # workgroups, partial sums in the scratch; 9-16 tokens on 64-160 tiles
    # the f16-MFMA kernel with K split, its partials in the scratch
    ((16, 2560, 6144, False), (5, 4096, 2560, True)),
    ((12, 2560, 6144, True), (3, 9728, 2560, False)),
    ((16, 9728, 2560, False), (9, 4096, 1024, True)),
])
def test_noalloc_matches_matvec(gpu, orc, first, second):
    for seed, (Mr, K, N, zeros) in enumerate((first, second)):
        c = orc.gptq_case(400 + seed, K, N, 128, zeros=zeros, M=Mr)
        w = sta.GptqWeight.upload(gpu, c["qweight"], c["scales"], 128, qzeros=c["qzeros"])
        x = torch.from_numpy(c["x"]).cuda()
        y_ref = torch.empty(Mr, N, device="cuda")
        y = torch.full((Mr, N), float("nan"), device="cuda")
        _mv(gpu, "st_gptq_i4_matvec", x, w, y_ref)
        _mv(gpu, "st_gptq_i4_matvec_noalloc", x, w, y)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), (Mr, K, N)
        ref = orc.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], K, N, 128, qzeros=c["qzeros"])
        assert orc.rel_l2(y.cpu().numpy(), ref) < TOL


def test_noalloc_rejects_beyond_scratch(gpu):
    """16 tokens of f32 x with K = 131072 need 8.4 MB of split rows, more
    than the 8 MiB scratch: a status, nothing launched, y untouched."""
    K, N, Mr = 131072, 64, 16
    x = torch.zeros(Mr, K, device="cuda")
    qw = torch.zeros(K // 8 * N, dtype=torch.int32, device="cuda")
    sc = torch.zeros(K // 128 * N, dtype=torch.float16, device="cuda")
    y = torch.full((Mr, N), 7.0, device="cuda")
    gpu.sync_stream()
    rc = lib().st_gptq_i4_matvec_noalloc(gpu.handle, x.data_ptr(), ST_F32, qw.data_ptr(), sc.data_ptr(), None, None,
                                         y.data_ptr(), Mr, K, N, 128, 0)
    torch.cuda.synchronize()
    assert rc == ST_ERR_WORKSPACE
    assert "scratch" in lib().st_last_error().decode()
    assert bool((y == 7.0).all())
