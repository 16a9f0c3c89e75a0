"""ll_decode_attention_noalloc (the entry point that allocates nothing)
against ll_decode_attention with a caller workspace, through the C ABI.

Two calls in a row, the second with a smaller input, each compared bit for
bit with the workspace entry point on the same inputs (same kernels, same
split plan), and with the oracle at the bf16 bar; a shape whose partials
exceed the scratch array is rejected before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import ops as O

pytestmark = pytest.mark.gpu


def _case(cuda, B, H, KVH, D, lens, seed):
    g = torch.Generator().manual_seed(seed)
    max_len = max(lens)
    P = B * max_len
    q = torch.randn(B, H, D, generator=g).bfloat16()
    pool = torch.randn(P, 2 * KVH, D, generator=g).bfloat16()
    perm = torch.from_numpy(np.random.RandomState(seed).permutation(P).astype(np.int32)).view(
        B, max_len)
    rids = list(range(B))
    ref = O.decode_attention(q, perm, rids, lens, pool[:, :KVH], pool[:, KVH:])
    return (q.to(cuda), pool.to(cuda), perm.to(cuda), torch.tensor(rids, dtype=torch.int32,
            device=cuda), torch.tensor(lens, dtype=torch.int64, device=cuda), max_len, ref)


def _call(L, noalloc, q, pool, r2t, rids, lens, max_len, KVH, ws=None):
    B, H, D = q.shape
    out = torch.full_like(q, float("nan"))
    k, v = pool[:, :KVH], pool[:, KVH:]
    head = (q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1), r2t.data_ptr(), r2t.stride(0),
            rids.data_ptr(), 0, lens.data_ptr(), 1, out.data_ptr(), out.stride(0), out.stride(1),
            B, H, KVH, D, max_len, ctypes.c_float(1.0 / D ** 0.5), 2)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = L.ll_decode_attention_noalloc(*head, stream)
    else:
        rc = L.ll_decode_attention(*head, ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, L.ll_last_error()
    torch.cuda.synchronize()
    return out


def test_noalloc_equals_workspace_entry_point(cuda):
    from lite_lang_amd import _lib
    L = _lib.load()
    cap = L.ll_decode_attention_noalloc_max_bytes()
    assert cap == 4 << 20
    shapes = [(40, 12, 2, 128, [600] * 40, 0),  # config 2
              (5, 16, 2, 128, [300, 17, 1, 250, 64], 1)]  # smaller, ragged, other heads
    for B, H, KVH, D, lens, seed in shapes:
        print(f"case: noalloc decode B={B} H={H} KVH={KVH} D={D} max_len={max(lens)}", flush=True)
        q, pool, r2t, rids, ln, max_len, ref = _case(cuda, B, H, KVH, D, lens, seed)
        need = L.ll_decode_attention_workspace_size(B, H, KVH, D, max_len)
        assert 0 < need <= cap
        ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
        want = _call(L, False, q, pool, r2t, rids, ln, max_len, KVH, ws)
        got = _call(L, True, q, pool, r2t, rids, ln, max_len, KVH)
        assert torch.equal(got, want)
        assert float((got.cpu().double() - ref).abs().max()) <= 2e-2
        again = _call(L, True, q, pool, r2t, rids, ln, max_len, KVH)  # tickets left at zero
        assert torch.equal(again, want)


def test_noalloc_rejects_shapes_beyond_its_scratch(cuda):
    from lite_lang_amd import _lib
    L = _lib.load()
    B, H, KVH, D, max_len = 64, 32, 8, 128, 65536
    assert L.ll_decode_attention_workspace_size(B, H, KVH, D, max_len) > \
        L.ll_decode_attention_noalloc_max_bytes()
    dummy = torch.zeros(16, dtype=torch.uint8, device=cuda)
    p = dummy.data_ptr()
    rc = L.ll_decode_attention_noalloc(p, 0, 0, p, 0, 0, p, 0, 0, p, 0, p, 0, p, 1, p, 0, 0,
                                       B, H, KVH, D, max_len, ctypes.c_float(0.1), 2,
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == -1 and b"scratch" in L.ll_last_error()
