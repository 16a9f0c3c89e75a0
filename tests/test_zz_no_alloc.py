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


_CAPTURE_SCRIPT = r"""
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, ROOT)
from lite_lang_amd import _lib
L = _lib.load()
dev = torch.device("cuda:0")
B, H, KVH, D, max_len = 40, 12, 2, 128, 600
rs = np.random.RandomState(9)
P = B * max_len
g = torch.Generator(device=dev).manual_seed(9)
q = torch.randn(B, H, D, device=dev, generator=g).bfloat16()
pool = torch.randn(P, 2 * KVH, D, device=dev, generator=g).bfloat16()
r2t = torch.from_numpy(rs.permutation(P).astype(np.int32)).view(B, max_len).to(dev)
rids = torch.arange(B, dtype=torch.int32, device=dev)
lens = torch.from_numpy(rs.randint(1, max_len + 1, size=B)).to(dev)
k, v = pool[:, :KVH], pool[:, KVH:]

def args(out):
    return (q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1), r2t.data_ptr(), r2t.stride(0),
            rids.data_ptr(), 0, lens.data_ptr(), 1, out.data_ptr(), out.stride(0), out.stride(1),
            B, H, KVH, D, max_len, ctypes.c_float(1.0 / D ** 0.5), 2)

torch.cuda.synchronize()
s = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
out = torch.zeros_like(q)
with torch.cuda.stream(s):
    with torch.cuda.graph(graph, stream=s):
        # the process's first no-alloc call: the scratch lookup happens here
        rc = L.ll_decode_attention_noalloc(*args(out), s.cuda_stream)
assert rc == 0, L.ll_last_error()
ws = torch.zeros(L.ll_decode_attention_workspace_size(B, H, KVH, D, max_len), dtype=torch.uint8,
                 device=dev)
want = torch.empty_like(q)
assert L.ll_decode_attention(*args(want), ws.data_ptr(), ws.numel(),
                             torch.cuda.current_stream().cuda_stream) == 0
torch.cuda.synchronize()
for rep in range(4):
    out.zero_()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {rep} differs"
    # eager no-alloc call between replays (shares the scratch array)
    again = torch.empty_like(q)
    assert L.ll_decode_attention_noalloc(*args(again), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(again, want)
print("capture ok", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(cuda):
    """In a fresh process, the first ll_decode_attention_noalloc call happens
    under graph capture (its scratch lookup queues no work, so nothing but the
    attention kernel is recorded); four replays, with eager no-alloc calls
    between them, each equal the workspace entry point bit for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("case: noalloc first call under capture (subprocess)", flush=True)
    res = subprocess.run([sys.executable, "-c", f"ROOT = {root!r}\n" + _CAPTURE_SCRIPT],
                         capture_output=True, text=True, timeout=180)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "capture ok" in res.stdout
