"""The C ABI library loads and exports every symbol the header declares.

No compute call is made here (this suite also runs on machines without a
GPU); only the host-side size queries are called.
"""
import ctypes

from lite_lang_amd import _lib


def test_header_symbols_are_exported_and_bound():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/litelang_amd.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(declared)
    assert lib.ll_version() == 1


def test_workspace_queries_are_host_only():
    lib = _lib.load()
    # decode attention: B=40, H=12, KVH=2, D=128, len 600
    n = lib.ll_decode_attention_workspace_size(40, 12, 2, 128, 600)
    assert n > 40 * 12 * 128 * 4
    assert lib.ll_argmax_workspace_size(40, 151936) > 0
    assert lib.ll_gemm_workspace_size(128, 2048, 2048) == 0


def test_null_arguments_are_rejected_before_launch():
    lib = _lib.load()
    rc = lib.ll_rmsnorm(None, 0, None, 0, None, None, 0, 4, 8, ctypes.c_float(1e-6), 2, None)
    assert rc == -1
    assert b"null pointer" in lib.ll_last_error()
    rc = lib.ll_gemm(None, 0, None, 0, None, None, 0, 4, 8, 8, 2, None, 0, None)
    assert rc == -1
