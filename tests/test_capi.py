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


def test_tile_gemm_rejects_short_row_strides():
    """The tile GEMM entry points check every row stride against its rows
    before any launch (a short ldy would make output rows overlap)."""
    lib = _lib.load()
    p = 256  # never dereferenced: the argument checks return first
    M, N, K = 256, 512, 128
    # ldx, ldw shorter than K; ldy shorter than N
    for bad in ((p, K - 8, p, K, None, p, N, M, N, K, 2, None),
                (p, K, p, K - 8, None, p, N, M, N, K, 2, None),
                (p, K, p, K, None, p, N - 4, M, N, K, 2, None)):
        assert lib.ll_gemm_tiled(*bad) == -1
        assert b"row strides" in lib.ll_last_error()
    # the gate/up forms (I = N / 2 outputs per row) and the int8 forms
    rc = lib.ll_gemm_gate_up_silu_tiled(p, K - 8, p, M, N // 2, K, 2, p, N // 2, None)
    assert rc == -1 and b"row strides" in lib.ll_last_error()
    rc = lib.ll_gemm_gate_up_silu_tiled(p, K, p, M, N // 2, K, 2, p, N // 2 - 4, None)
    assert rc == -1 and b"row strides" in lib.ll_last_error()
    i8 = lib.ll_gemm_i8_i32_tiled(p, K, p, K, p, N - 4, M, N, K, None)
    assert i8 == -1 and b"row strides" in lib.ll_last_error()


def test_host_only_settings():
    lib = _lib.load()
    assert lib.ll_decode_sync_error_offset() > 0
    assert lib.ll_decode_sync_error_offset() + 4 <= lib.ll_decode_sync_bytes()
    assert lib.ll_decode_sync_set_spin_limit(-(1 << 21)) == -1
    assert lib.ll_decode_sync_set_spin_limit(0) == 0
    prev = lib.ll_decode_attention_set_same_launch_merge(0)
    assert lib.ll_decode_attention_set_same_launch_merge(prev) == 0
    rc = lib.ll_argmax_status(256, 8, 4, 8, 256, None, 0, 2, None, None)
    assert rc == -1 and b"status" in lib.ll_last_error()
    rc = lib.ll_embedding_rmsnorm_epoch(256, 8, 8, 256, 0, 256, 8, 256, 256, 8, 4, 8,
                                        _lib.F32(1e-6), 2, None, None, 0, None, None, None, None)
    assert rc == -1 and b"epoch" in lib.ll_last_error()
    # a slot-table update without its slots, rows and columns
    rc = lib.ll_embedding_rmsnorm_epoch(256, 8, 8, 256, 0, 256, 8, 256, 256, 8, 4, 8,
                                        _lib.F32(1e-6), 2, 256, 256, 8, None, 256, 256, None)
    assert rc == -1 and b"slot-table" in lib.ll_last_error()
