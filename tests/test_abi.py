"""CPU checks of the C ABI: the header compiles as C and C++, the library
loads, every declared symbol is exported, the ctypes table matches the
header, and argument errors come back as status codes, not crashes."""
import ctypes
import os
import subprocess

import pytest

import shady_thinker_amd as sta
from shady_thinker_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_header_compiles_as_c_and_cpp(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "shady_hip.h"\nint main(void){return ST_OK;}\n')
    for cc in (["gcc", "-std=c99"], ["g++", "-x", "c++", "-std=c++11"]):
        subprocess.run([*cc, "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"), str(src)],
                       check=True)


def test_library_exports_every_header_symbol():
    L = sta.lib()
    names = _lib.header_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    assert sorted(_lib._SIGNATURES) == sorted(_lib.header_symbols())


def test_version_and_error_string():
    L = sta.lib()
    assert L.st_version().decode().startswith("shady_hip")
    assert isinstance(L.st_last_error(), bytes)


def test_null_arguments_are_rejected():
    L = sta.lib()
    assert L.st_context_create(0, None) == 1  # ST_ERR_INVALID
    assert b"NULL" in L.st_last_error()
    for fn, nargs in [("st_gptq_i4_matvec", 13), ("st_gptq_i4_silu_matvec", 13), ("st_gptq_i4_gate_up_silu", 16),
                      ("st_int8_matvec", 10), ("st_gptq_i4_gemm", 13), ("st_gptq_i4_silu_gemm", 14), ("st_gptq_i4_dequant", 11),
                      ("st_gptq_i4_act_order", 8), ("st_bf16_matvec", 8), ("st_int8_repack", 5),
                      ("st_gptq_i4_repack", 6)]:
        args = [None] * nargs
        rc = getattr(L, fn)(*[0 if t in (ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t) else None
                               for t in getattr(L, fn).argtypes])
        assert rc == 1, fn
    assert L.st_flush(None) == 1
    assert L.st_context_destroy(None) == 0


def test_context_create_without_gpu_reports_hip_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    rc = sta.lib().st_context_create(0, ctypes.byref(h))
    assert rc == 5  # ST_ERR_HIP
    assert sta.lib().st_last_error()
    with pytest.raises(sta.ShadyHipError):
        _lib.call("st_context_create", 0, ctypes.byref(h))


def test_quant_config_parsing(tmp_path):
    p = tmp_path / "quantize_config.json"
    p.write_text('{"bits": 4, "group_size": 64, "quant_method": "gptq", "sym": false}')
    qc = sta.QuantConfig.from_file(str(p))
    assert (qc.bits, qc.group_size, qc.quant_method, qc.sym) == (4, 64, "gptq", False)
    assert sta.QuantConfig.from_dict({}).group_size == 128
