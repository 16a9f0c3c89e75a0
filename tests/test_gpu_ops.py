"""GPU parity of every kernel against the CPU oracle (oracle/ops.py).

Tolerances: outputs stored in bf16/fp16 are compared with the float64
oracle evaluated on the same (rounded) inputs at max-abs 2e-2 (the bar the
north star sets for bf16 attention, norm and logits); fp32 outputs at 1e-4.
Integer / index outputs are compared exactly.
"""
import math

import numpy as np
import pytest
import torch

from oracle import ops as O

pytestmark = pytest.mark.gpu

BF16_ATOL = 2e-2
F32_ATOL = 1e-4
# GEMM and SiLU outputs grow with |y| (K-term sums, products of N(0,1)):
# their bf16 storage alone rounds by up to half an ulp = 2^-9 |y|, so they are
# checked at |a - b| <= 2e-2 + 2^-7 |b| (one bf16 ulp relative).
BF16_RTOL = 2.0 ** -7


def _ops():
    from lite_lang_amd import ops
    return ops


def _tol(dtype):
    return F32_ATOL if dtype == torch.float32 else BF16_ATOL


def _maxdiff(a, b):
    return float((a.detach().cpu().to(torch.float64) - b.to(torch.float64)).abs().max())


def _close_rel(a, b, atol=BF16_ATOL, rtol=BF16_RTOL):
    a = a.detach().cpu().to(torch.float64)
    b = b.to(torch.float64)
    excess = (a - b).abs() - (atol + rtol * b.abs())
    return float(excess.max()) <= 0.0


# ------------------------------------------------------------ decode attention
def _decode_case(cuda, B, H, KVH, D, lens, dtype, seed, pool_slots=None, rids=None):
    g = torch.Generator().manual_seed(seed)
    max_len = max(lens)
    P = pool_slots or B * max_len
    q = torch.randn(B, H, D, generator=g).to(dtype)
    pool = torch.randn(P, 2 * KVH, D, generator=g).to(dtype)
    perm = torch.from_numpy(np.random.RandomState(seed).permutation(P)[: B * max_len]
                            .astype(np.int32)).view(B, max_len)
    r2t = torch.zeros(B + 3, max_len, dtype=torch.int32)
    rids = rids if rids is not None else list(range(B))
    for b, r in enumerate(rids):
        r2t[r] = perm[b]
    ref = O.decode_attention(q, r2t, rids, lens, pool[:, :KVH], pool[:, KVH:])
    qd, pd, r2td = q.to(cuda), pool.to(cuda), r2t.to(cuda)
    out = torch.empty_like(qd)
    _ops().decode_attention(qd, r2td, torch.tensor(rids, dtype=torch.int32, device=cuda),
                            torch.tensor(lens, dtype=torch.int64, device=cuda), max_len,
                            pd[:, :KVH], pd[:, KVH:], out)
    torch.cuda.synchronize()
    return out, ref


def test_decode_attention_config2_uniform(cuda):
    print("case: decode config2 B=40 ctx=600 H=12 KVH=2 D=128 bf16", flush=True)
    out, ref = _decode_case(cuda, 40, 12, 2, 128, [600] * 40, torch.bfloat16, 0)
    assert _maxdiff(out, ref) <= BF16_ATOL


def test_decode_attention_config2_varlen(cuda):
    lens = np.random.RandomState(1).randint(1, 601, size=40).tolist()
    print(f"case: decode config2b varlen lens[:5]={lens[:5]}", flush=True)
    out, ref = _decode_case(cuda, 40, 12, 2, 128, lens, torch.bfloat16, 1)
    assert _maxdiff(out, ref) <= BF16_ATOL


@pytest.mark.parametrize("B,L,splits", [(4, 8000, 16), (7, 3000, 16), (32, 600, 2), (40, 656, 3)])
def test_decode_attention_split_counts(cuda, B, L, splits):
    """Shapes on either side of the split-count rule (head_dim 128): at most
    16 splits from 8 (sequence, KV head) units up (4 x 8000 tokens would
    fill a dispatch round with 32, 7 x 3000 with 18; more than 8 splits merge
    by ticket), and from 64 units up the count the cost fit picks (2 splits
    at 32 x 600, 3 at 40 x 656). Each against the oracle."""
    from lite_lang_amd import _lib
    assert _lib.load().ll_decode_attention_split_count(B, 2, 128, L) == splits
    lens = [L] * B
    lens[0] = L - 5  # one shorter row: its last split holds fewer tiles
    print(f"case: decode split count B={B} L={L} splits={splits}", flush=True)
    out, ref = _decode_case(cuda, B, 16, 2, 128, lens, torch.bfloat16, 7)
    assert _maxdiff(out, ref) <= BF16_ATOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("H,KVH,D", [(16, 2, 128), (8, 8, 64), (4, 2, 64), (6, 1, 128)])
def test_decode_attention_shapes(cuda, dtype, H, KVH, D):
    lens = [1, 33, 100, 257, 31, 64]
    print(f"case: decode H={H} KVH={KVH} D={D} {dtype}", flush=True)
    out, ref = _decode_case(cuda, len(lens), H, KVH, D, lens, dtype, 2, rids=[4, 0, 2, 1, 3, 5])
    assert _maxdiff(out, ref) <= _tol(dtype)


def test_decode_attention_repeat_calls_are_identical(cuda):
    # the last split of each (sequence, KV head) merges the others' partial
    # words, whose zero means "not yet written", and zeroes the rows it merged:
    # calls of different shapes and split counts in a row share one workspace,
    # must not interfere (no call may take an earlier call's words), and leave
    # the whole workspace at zero
    print("case: decode repeat, interleaved shapes", flush=True)
    a, ref = _decode_case(cuda, 40, 16, 2, 128, [700] * 40, torch.bfloat16, 3)
    c, cref = _decode_case(cuda, 2, 16, 2, 128, [40, 2000], torch.bfloat16, 4)
    d, dref = _decode_case(cuda, 40, 12, 2, 128, [600] * 40, torch.bfloat16, 0)
    e, eref = _decode_case(cuda, 64, 8, 8, 64, [300] * 64, torch.float16, 6)
    b, _ = _decode_case(cuda, 40, 16, 2, 128, [700] * 40, torch.bfloat16, 3)
    assert torch.equal(a, b)
    for out, r in ((a, ref), (c, cref), (d, dref), (e, eref)):
        assert _maxdiff(out, r) <= BF16_ATOL
    ws = _ops()._WS[_ops()._ws_key(cuda, "decode_attention")]
    assert int(ws[:16384].count_nonzero()) == 0, "split tickets not back at zero"
    assert int(ws.count_nonzero()) == 0, "split partials not back at zero"


def test_decode_attention_reference_wrapper(cuda):
    from lite_lang_amd.kernel.develop_flash_attn.flash_decoding import (
        token_decode_attention_flash_decoding)
    g = torch.Generator().manual_seed(5)
    B, H, KVH, D = 3, 8, 2, 64
    lens = [1000, 2000, 3000]  # test_flash_decoding shape (flash_decoding.py:315-345)
    P = sum(lens)
    q = torch.randn(B, H, D, generator=g).half()
    k = torch.randn(P, KVH, D, generator=g).half()
    v = torch.randn(P, KVH, D, generator=g).half()
    r2t = torch.zeros(B, max(lens), dtype=torch.int32)
    s = 0
    for i, l in enumerate(lens):
        r2t[i, :l] = torch.arange(s, s + l)
        s += l
    ref = O.decode_attention(q, r2t, list(range(B)), lens, k, v)
    out = torch.empty(B, H, D, dtype=torch.float16, device=cuda)
    token_decode_attention_flash_decoding(q.to(cuda), r2t.to(cuda), torch.arange(B, device=cuda),
                                          torch.tensor(lens, device=cuda), max(lens), H, D,
                                          k.to(cuda), v.to(cuda), out)
    torch.cuda.synchronize()
    assert _maxdiff(out, ref) <= 1e-2  # the reference test's own atol


# ------------------------------------------------------------ prefill attention
def _prefill_case(cuda, H, KVH, D, lens, shared, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    qlens = [l - s for l, s in zip(lens, shared)]
    T = sum(qlens)
    starts = np.concatenate([[0], np.cumsum(qlens)[:-1]]).tolist()
    P = sum(lens) + 17
    q = torch.randn(T, H, D, generator=g).to(dtype)
    pool = torch.randn(P, 2 * KVH, D, generator=g).to(dtype)
    perm = np.random.RandomState(seed).permutation(P).astype(np.int32)
    r2t = torch.zeros(B + 1, max(lens), dtype=torch.int32)
    rids = list(range(1, B + 1))
    o = 0
    for b, r in enumerate(rids):
        r2t[r, :lens[b]] = torch.from_numpy(perm[o:o + lens[b]])
        o += lens[b]
    ref = O.prefill_attention(q, pool[:, :KVH], pool[:, KVH:], rids, starts, lens, r2t,
                              b_shared_seq_len=shared,
                              p_dtype=None if dtype == torch.float32 else dtype)
    pd = pool.to(cuda)
    out = torch.empty(T, H, D, dtype=dtype, device=cuda)
    _ops().prefill_attention(q.to(cuda), pd[:, :KVH], pd[:, KVH:], out,
                             torch.tensor(rids, dtype=torch.int32, device=cuda),
                             torch.tensor(starts, dtype=torch.int64, device=cuda),
                             torch.tensor(lens, dtype=torch.int64, device=cuda), max(lens),
                             r2t.to(cuda),
                             b_shared_seq_len=torch.tensor(shared, device=cuda) if any(shared) else None)
    torch.cuda.synchronize()
    return out, ref


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("H,KVH,D", [(16, 2, 128), (4, 4, 64)])
def test_prefill_attention_varlen(cuda, dtype, H, KVH, D):
    lens = [1, 70, 200, 64, 129]
    print(f"case: prefill H={H} KVH={KVH} D={D} {dtype}", flush=True)
    out, ref = _prefill_case(cuda, H, KVH, D, lens, [0] * len(lens), dtype, 10)
    assert _maxdiff(out, ref) <= _tol(dtype)


@pytest.mark.parametrize("H,KVH,lens,shared", [
    (28, 4, [600, 129, 1, 257], [0, 0, 0, 0]),     # odd group (7 q heads per KV head)
    (12, 2, [700, 333, 64], [0, 0, 0]),           # 1.5B geometry, several 128-row blocks
    (16, 2, [650, 400, 90], [520, 17, 89]),       # long cached prefixes, one-row query
    (16, 2, [1100, 257], [0, 0])])                # 3B geometry, rows past 1024
def test_prefill_attention_long_and_odd_groups(cuda, H, KVH, lens, shared):
    print(f"case: prefill H={H} KVH={KVH} lens={lens} shared={shared}", flush=True)
    out, ref = _prefill_case(cuda, H, KVH, 128, lens, shared, torch.bfloat16, 12)
    assert _maxdiff(out, ref) <= _tol(torch.bfloat16)


@pytest.mark.parametrize("H,KVH", [(16, 2), (12, 2)])
def test_prefill_attention_growing_scores(cuda, H, KVH):
    """Keys scaled up tile after tile, so the running maxima jump by far more
    than 2^8 in the exp2 domain at several tiles (the kernel's rescale path),
    with rows that also see a prompt-cache prefix."""
    g = torch.Generator().manual_seed(13)
    lens, shared = [700, 300, 64], [100, 0, 0]
    B = len(lens)
    qlens = [l - s for l, s in zip(lens, shared)]
    starts = np.concatenate([[0], np.cumsum(qlens)[:-1]]).tolist()
    P = sum(lens) + 5
    q = torch.randn(sum(qlens), H, 128, generator=g).bfloat16()
    pool = torch.randn(P, 2 * KVH, 128, generator=g)
    r2t = torch.zeros(B, max(lens), dtype=torch.int32)
    o = 0
    for b in range(B):
        r2t[b, :lens[b]] = torch.arange(o, o + lens[b], dtype=torch.int32)
        # key j of the request (tile j // 64) scaled by 1 + 2 (j // 64)
        pool[o:o + lens[b], :KVH] *= (1 + 2 * (torch.arange(lens[b]) // 64)).float()[:, None, None]
        o += lens[b]
    pool = pool.bfloat16()
    rids = list(range(B))
    ref = O.prefill_attention(q, pool[:, :KVH], pool[:, KVH:], rids, starts, lens, r2t,
                              b_shared_seq_len=shared, p_dtype=torch.bfloat16)
    pd = pool.to(cuda)
    out = torch.empty_like(q, device=cuda)
    print(f"case: prefill growing scores H={H} KVH={KVH}", flush=True)
    _ops().prefill_attention(q.to(cuda), pd[:, :KVH], pd[:, KVH:], out,
                             torch.tensor(rids, dtype=torch.int32, device=cuda),
                             torch.tensor(starts, dtype=torch.int64, device=cuda),
                             torch.tensor(lens, dtype=torch.int64, device=cuda), max(lens),
                             r2t.to(cuda), b_shared_seq_len=torch.tensor(shared, device=cuda))
    torch.cuda.synchronize()
    assert _maxdiff(out, ref) <= _tol(torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prefill_attention_prompt_cache(cuda, dtype):
    # shapes of test_context_attention_with_kv_cache_and_prompt_cache
    # (flash_attn_v2.py:765-800) plus a long-prefix case
    lens, shared = [16, 32, 300], [8, 11, 260]
    print(f"case: prefill prompt cache {dtype}", flush=True)
    out, ref = _prefill_case(cuda, 8, 2, 64, lens, shared, dtype, 11)
    assert _maxdiff(out, ref) <= _tol(dtype)


@pytest.mark.parametrize("H,KVH,B,maxlen,with_shared", [
    (16, 2, 300, 260, False),   # 3B geometry: ~1,600 items over 256 workgroups
    (28, 4, 120, 300, True)])   # odd group (128-row blocks), prompt-cache prefixes
def test_prefill_attention_many_items_per_workgroup(cuda, H, KVH, B, maxlen, with_shared):
    """Batches with far more work items (row block, request, KV head, head
    group) than workgroups, so that each persistent workgroup streams several
    items back to back, ragged lengths leaving many items empty."""
    rs = np.random.RandomState(14)
    lens = rs.randint(1, maxlen + 1, size=B).tolist()
    shared = [int(rs.randint(0, l)) if with_shared and b % 3 == 0 else 0
              for b, l in enumerate(lens)]
    print(f"case: prefill many items H={H} KVH={KVH} B={B}", flush=True)
    out, ref = _prefill_case(cuda, H, KVH, 128, lens, shared, torch.bfloat16, 15)
    assert _maxdiff(out, ref) <= _tol(torch.bfloat16)


def test_prefill_attention_grid_past_64_passes(cuda):
    """16,800 work items: more than 64 per CU, so the grid grows past one
    workgroup per CU. Bit-identical to the same requests launched 16 at a
    time, where every workgroup takes a single item."""
    H, KVH, D, B = 4, 4, 64, 4200
    rs = np.random.RandomState(16)
    lens = rs.randint(1, 41, size=B)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    T = int(lens.sum())
    g = torch.Generator().manual_seed(16)
    q = torch.randn(T, H, D, generator=g).bfloat16().to(cuda)
    pool = torch.randn(T + 8, 2 * KVH, D, generator=g).bfloat16().to(cuda)
    r2t = torch.zeros(B, 40, dtype=torch.int32)
    perm = torch.from_numpy(rs.permutation(T + 8).astype(np.int32))
    for b in range(B):
        r2t[b, :lens[b]] = perm[starts[b]:starts[b] + lens[b]]
    r2t = r2t.to(cuda)
    rids = torch.arange(B, dtype=torch.int32, device=cuda)
    st = torch.from_numpy(starts).to(cuda)
    ln = torch.from_numpy(lens).to(cuda)
    ops = _ops()
    print("case: prefill grid past 64 passes", flush=True)
    whole = torch.empty_like(q)
    ops.prefill_attention(q, pool[:, :KVH], pool[:, KVH:], whole, rids, st, ln, 40, r2t)
    parts = torch.empty_like(q)
    for b0 in range(0, B, 16):
        ops.prefill_attention(q, pool[:, :KVH], pool[:, KVH:], parts, rids[b0:b0 + 16],
                              st[b0:b0 + 16], ln[b0:b0 + 16], 40, r2t)
    torch.cuda.synchronize()
    assert torch.equal(whole, parts)


# ------------------------------------------------------------ elementwise
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rmsnorm_and_residual(cuda, dtype):
    g = torch.Generator().manual_seed(20)
    x = (torch.randn(37, 2048, generator=g) * 0.5 + 0.3).to(dtype)
    r = torch.randn(37, 2048, generator=g).to(dtype)
    gamma = (torch.rand(2048, generator=g) + 0.5).to(dtype)
    ops = _ops()
    out = ops.rmsnorm(x.to(cuda), gamma.to(cuda), 1e-6)
    assert _maxdiff(out, O.rmsnorm(x, gamma, 1e-6)) <= _tol(dtype)
    xd = x.to(cuda)
    out2 = ops.rmsnorm(xd, gamma.to(cuda), 1e-5, residual=r.to(cuda))
    h = O.rnd(x.double() + r.double(), dtype)
    assert torch.equal(xd.cpu(), h.to(dtype))  # residual stored exactly as dtype(x + r)
    assert _maxdiff(out2, O.rmsnorm(h, gamma, 1e-5)) <= _tol(dtype)


def test_rmsnorm_reference_wrapper(cuda):
    from lite_lang_amd.kernel.develop_rmsnorm.rms_norm import rmsnorm
    g = torch.Generator().manual_seed(21)
    # test_rmsnorm shape and distribution (rms_norm.py:101-113)
    x = torch.normal(0.3, 0.5, size=(100, 2048), generator=g)
    gamma = torch.normal(0.3, 0.5, size=(2048,), generator=g)
    out = rmsnorm(x.to(cuda), gamma.to(cuda), 1e-5)
    assert _maxdiff(out, O.rmsnorm(x, gamma, 1e-5)) <= 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rotary_emb_wrapper_on_pool_view(cuda, dtype):
    from lite_lang_amd.kernel.develop_rope.rope import rotary_emb_fwd
    g = torch.Generator().manual_seed(22)
    T, H, KVH, D = 50, 16, 2, 128
    q = (torch.randn(T, H, D, generator=g) * 0.3).to(dtype)
    kv = (torch.randn(T, 2 * KVH, D, generator=g) * 0.3).to(dtype)
    cos = torch.randn(T, D // 2, generator=g).clamp(-1, 1).to(dtype)
    sin = torch.randn(T, D // 2, generator=g).clamp(-1, 1).to(dtype)
    qd, kvd = q.to(cuda), kv.to(cuda)
    rotary_emb_fwd(qd, kvd[:, :KVH], cos.to(cuda), sin.to(cuda))
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert _maxdiff(qd, O.rotary(q, cos, sin)) <= tol
    assert _maxdiff(kvd[:, :KVH], O.rotary(kv[:, :KVH], cos, sin)) <= tol
    assert torch.equal(kvd[:, KVH:].cpu(), kv[:, KVH:])  # V heads untouched


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_kv_scatter(cuda, dtype):
    g = torch.Generator().manual_seed(23)
    T, H, KVH, D, P = 19, 4, 2, 64, 64
    qkv = torch.randn(T, (H + 2 * KVH) * D, generator=g).to(dtype)
    pos = torch.randint(0, 100, (T,), generator=g)
    cos, sin = O.rope_table(128, D)
    slots = torch.from_numpy(np.random.RandomState(3).permutation(P)[:T].astype(np.int32))
    pool = torch.zeros(P, 2 * KVH, D, dtype=dtype)
    qkvd, poold = qkv.to(cuda), pool.to(cuda)
    _ops().rope_kv_scatter(qkvd, H, KVH, D, pos.to(cuda), cos.float().to(cuda),
                           sin.float().to(cuda), slots.to(cuda), poold)
    torch.cuda.synchronize()
    c, s = cos[pos], sin[pos]
    q_ref = O.rotary(qkv[:, :H * D].view(T, H, D), c, s)
    k_ref = O.rotary(qkv[:, H * D:(H + KVH) * D].view(T, KVH, D), c, s)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert _maxdiff(qkvd[:, :H * D].view(T, H, D), q_ref) <= tol
    assert _maxdiff(poold[slots.long(), :KVH], k_ref) <= tol
    assert torch.equal(poold[slots.long(), KVH:].cpu(), qkv[:, (H + KVH) * D:].view(T, KVH, D))
    untouched = torch.ones(P, dtype=torch.bool)
    untouched[slots.long()] = False
    assert float(poold[untouched.to(cuda)].abs().max()) == 0.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_silu_and_mul_in_place(cuda, dtype):
    from lite_lang_amd.kernel.develop_silu_and_mul.silu_and_mul import silu_and_mul_fwd
    g = torch.Generator().manual_seed(24)
    x = torch.randn(40, 2 * 1376, generator=g).to(dtype)
    xd = x.to(cuda)
    out = silu_and_mul_fwd(xd)
    assert out.data_ptr() == xd.data_ptr() and out.stride(0) == 2 * 1376
    ref = O.silu_and_mul(x, dtype)
    if dtype == torch.float32:
        assert _maxdiff(out, ref) <= 1e-5
    else:
        assert _close_rel(out, ref)


def test_embedding_and_argmax(cuda):
    g = torch.Generator().manual_seed(25)
    table = torch.randn(1000, 64, generator=g).bfloat16()
    ids = torch.randint(0, 1000, (33,), generator=g)
    out = _ops().embedding(table.to(cuda), ids.to(cuda))
    assert torch.equal(out.cpu(), table[ids])
    logits = torch.randn(40, 151936, generator=g).bfloat16()
    logits[3, 100] = 50.0
    logits[3, 90000] = 50.0  # tie across chunks: first index wins
    logits[7, :] = 1.0       # all equal
    got = _ops().argmax(logits.to(cuda)).cpu()
    assert torch.equal(got, O.argmax_first(logits.float()))
    assert got[3] == 100 and got[7] == 0
    got2 = _ops().argmax(logits[:, :5000].contiguous().to(cuda)).cpu()  # single-chunk path
    assert torch.equal(got2, O.argmax_first(logits[:, :5000].float()))
    # ties inside one 16-byte load and across the 8192-wide chunk boundary,
    # fp16, and a width that is not a multiple of 8 (the scalar pass)
    lg = torch.randn(12, 20001, generator=g).half()
    lg[5, 16:24] = 60.0
    lg[9, 8191] = 70.0
    lg[9, 8192] = 70.0
    lg[10, 20000] = 80.0
    for width in (20000, 20001):
        sub = lg[:, :width].contiguous()
        got3 = _ops().argmax(sub.to(cuda)).cpu()
        assert torch.equal(got3, O.argmax_first(sub.float())), width
    assert got3[5] == 16 and got3[9] == 8191 and got3[10] == 20000


# ------------------------------------------------------------ GEMM
@pytest.mark.parametrize("M,N,K", [(1, 2560, 2048), (40, 2560, 2048), (40, 2048, 11008),
                                   (64, 300, 688), (40, 22016, 2048), (300, 520, 264),
                                   (129, 256, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_mfma(cuda, M, N, K, dtype):
    g = torch.Generator().manual_seed(30)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) * 0.02).to(dtype)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype)
    print(f"case: gemm M={M} N={N} K={K} {dtype}", flush=True)
    y = _ops().gemm(x.to(cuda), w.to(cuda), b.to(cuda))
    torch.cuda.synchronize()
    ref = O.linear(x, w, b)
    assert _close_rel(y, ref)


def test_gemm_fp32_and_strided_input(cuda):
    g = torch.Generator().manual_seed(31)
    x = torch.randn(17, 2 * 96, generator=g)
    w = torch.randn(70, 96, generator=g)
    y = _ops().gemm(x.to(cuda)[:, :96], w.to(cuda))
    assert _maxdiff(y, O.linear(x[:, :96], w)) <= 1e-4
    xb = x.bfloat16().to(cuda)
    yb = _ops().gemm(xb[:, 96:], w.bfloat16().to(cuda))
    assert _close_rel(yb, O.linear(x[:, 96:].bfloat16(), w.bfloat16()))


# ------------------------------------------------------------ slot table on device
def test_page_cache_kat_on_device(cuda):
    import json, os
    from lite_lang_amd.models.cache import PageCache
    kat = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "page_cache_kat.json")))
    pc = PageCache(kat["max_batch_size"], kat["max_length"], 0.0, 1, 128, 2,
                   torch_dtype=torch.bfloat16, kv_max_size=4096, device=cuda)
    rids = [pc.alloc_req(), pc.alloc_req()]
    lens = kat["prefill"]["seq_lens"]
    got = pc.alloc_token_idxs(rids, [0, 0], lens)
    r2t = pc.req_to_tokens_.cpu()
    assert torch.cat([r2t[r, :l] for r, l in zip(rids, lens)]).tolist() == \
        kat["prefill"]["expected_rows_concat"]
    assert got.cpu().tolist() == list(range(7))
    pc.alloc_token_idxs(rids, lens, kat["decode"]["new_tokens"])
    r2t = pc.req_to_tokens_.cpu()
    assert torch.cat([r2t[0, :3], r2t[1, :6]]).tolist() == kat["decode"]["expected_rows_concat"]


# ------------------------------------------------------------ decode split-K path
def _splitk(cuda, M, N, K, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) * 0.02).to(dtype)
    ops = _ops()
    s = ops.gemm_splitk_count(M, N, K)
    part = torch.zeros(s * M * N + 64, dtype=torch.float32, device=cuda)
    s2 = ops.gemm_splitk(x.to(cuda), w.to(cuda), part)
    torch.cuda.synchronize()
    assert s2 == s
    return x, w, part, s


@pytest.mark.parametrize("M,N,K", [(40, 2560, 2048), (40, 2048, 2048), (40, 22016, 2048),
                                   (40, 2048, 11008), (1, 4096, 1024), (64, 6000, 640),
                                   (17, 512, 688)])
def test_gemm_splitk_partials_sum_to_product(cuda, M, N, K):
    print(f"case: gemm_splitk M={M} N={N} K={K}", flush=True)
    x, w, part, s = _splitk(cuda, M, N, K, 40)
    total = part[: s * M * N].view(s, M, N).sum(0).cpu().double()
    ref = O.linear(x, w)
    assert float((total - ref).abs().max()) <= 1e-4 * max(1.0, float(ref.abs().max()))


@pytest.mark.parametrize("M,N,K", [(40, 8192, 2048), (3, 151936, 256)])
def test_gemm_wide_n_lds_path(cuda, M, N, K):
    g = torch.Generator().manual_seed(41)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    b = (torch.randn(N, generator=g) * 0.1).bfloat16()
    print(f"case: gemm wide M={M} N={N} K={K}", flush=True)
    y = _ops().gemm(x.to(cuda), w.to(cuda), b.to(cuda))
    assert _close_rel(y, O.linear(x, w, b))


# ------------------------------------------------------------ packed weights
def _pack_reference(w, tr=64):
    """Host restatement of the ll_gemm_pack layout with tr-row tiles: block
    (kc, t) of tr * 256 bytes holds rows tr*t + 4ii + lane//16, 16 B chunk
    (lane % 16) ^ (row % 16) of the 128-column chunk kc, at unit 64 ii + lane;
    blocks kc-major; rows >= N zero."""
    N, K = w.shape
    T = -(-N // tr)
    wp = torch.zeros(T * tr, K, dtype=w.dtype)
    wp[:N] = w
    u = wp.view(torch.int16).numpy().reshape(T, tr, K // 128, 16, 8)  # [t, r, kc, chunk, 8]
    ii, lane = np.meshgrid(np.arange(tr // 4), np.arange(64), indexing="ij")
    r = 4 * ii + lane // 16
    c = (lane % 16) ^ (r % 16)
    blocks = u[:, r, :, c, :]  # advanced indices split by a slice lead: [tr/4, 64, t, kc, 8]
    return torch.from_numpy(np.ascontiguousarray(blocks.transpose(3, 2, 0, 1, 4))).reshape(-1)


def _tile_rows(N, K):
    from lite_lang_amd import _lib
    return _lib.load().ll_gemm_packed_tile_rows(N, K)


@pytest.mark.parametrize("N,K,tr", [(200, 256, 64), (128, 128, 64), (2560, 2048, 64),
                                    (16500, 256, 128), (17000, 384, 128)])
def test_gemm_pack_layout(cuda, N, K, tr):
    g = torch.Generator().manual_seed(45)
    w = torch.randn(N, K, generator=g).bfloat16()
    print(f"case: gemm_pack N={N} K={K}", flush=True)
    assert _tile_rows(N, K) == tr  # one split over > 256 64-row tiles -> 128-row tiles
    wp = _ops().pack_weight(w.to(cuda))
    torch.cuda.synchronize()
    got = wp.data.cpu().view(torch.int16)
    assert torch.equal(got, _pack_reference(w, tr))


@pytest.mark.parametrize("M,N,K", [(40, 2560, 2048), (40, 2048, 11008), (1, 22016, 2048),
                                   (64, 200, 384), (17, 4096, 1024)])
def test_gemm_splitk_packed(cuda, M, N, K):
    print(f"case: gemm_splitk_packed M={M} N={N} K={K}", flush=True)
    x, w, part, s = _splitk(cuda, M, N, K, 46)
    wp = _ops().pack_weight(w.to(cuda))
    part2 = torch.full_like(part, float("nan"))
    s2 = _ops().gemm_splitk_packed(x.to(cuda), wp, part2)
    torch.cuda.synchronize()
    assert s2 == s
    total = part2[: s * M * N].view(s, M, N).sum(0).cpu().double()
    ref = O.linear(x, w)
    assert float((total - ref).abs().max()) <= 1e-4 * max(1.0, float(ref.abs().max()))
    # same splits as the unpacked kernel: each split's partial agrees to fp32 rounding
    a = part[: s * M * N].view(s, M, N).cpu().double()
    b = part2[: s * M * N].view(s, M, N).cpu().double()
    assert float((a - b).abs().max()) <= 1e-5 * max(1.0, float(a.abs().max()))


@pytest.mark.parametrize("M,N,K", [(40, 151936, 2048), (3, 1000, 256)])
def test_gemm_packed_with_bias(cuda, M, N, K):
    g = torch.Generator().manual_seed(47)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    b = (torch.randn(N, generator=g) * 0.1).bfloat16()
    print(f"case: gemm_packed M={M} N={N} K={K}", flush=True)
    y = _ops().gemm_packed(x.to(cuda), _ops().pack_weight(w.to(cuda)), b.to(cuda))
    assert _close_rel(y, O.linear(x, w, b))


@pytest.mark.parametrize("M,I,K", [(40, 11008, 2048), (64, 11008, 256), (40, 12300, 256), (1, 256, 128),
                                    (64, 200, 384), (17, 4864, 896 + 128)])
def test_gate_up_silu_fused_equals_unfused(cuda, M, I, K):
    """The fused epilogue rounds exactly as gemm_splitk + silu_and_mul_splitk do
    with one split: bit-identical output; and within tolerance of the oracle."""
    g = torch.Generator().manual_seed(48)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(2 * I, K, generator=g) * 0.02).bfloat16()
    print(f"case: gate_up_silu M={M} I={I} K={K}", flush=True)
    ops = _ops()
    xd, wd = x.to(cuda), w.to(cuda)
    fused = ops.gate_up_silu(xd, ops.pack_gate_up(wd))
    s = ops.gemm_splitk_count(M, 2 * I, K)
    part = torch.zeros(s * M * 2 * I, dtype=torch.float32, device=cuda)
    ops.gemm_splitk_packed(xd, ops.pack_weight(wd), part)
    unfused = torch.empty(M, I, dtype=torch.bfloat16, device=cuda)
    ops.silu_and_mul_splitk(part, s, unfused)
    torch.cuda.synchronize()
    if s == 1:  # the same fp32 sums reach the same rounding steps
        assert torch.equal(fused, unfused)
    ref = O.silu_and_mul(O.rnd(O.linear(x, w), torch.bfloat16), torch.bfloat16)
    assert _close_rel(fused, ref)


@pytest.mark.parametrize("I,K,tr", [(70, 256, 64), (8200, 128, 96), (12300, 128, 128)])
def test_gate_up_pack_layout(cuda, I, K, tr):
    from lite_lang_amd import _lib
    g = torch.Generator().manual_seed(49)
    w = torch.randn(2 * I, K, generator=g).bfloat16()
    print(f"case: gate_up pack I={I} K={K}", flush=True)
    assert _lib.load().ll_gemm_packed_gate_up_tile_rows(I) == tr
    wp = _ops().pack_gate_up(w.to(cuda))
    torch.cuda.synchronize()
    half = tr // 2
    T = -(-I // half)
    # interleaved row order: tile t = gate rows half*t.., then the same up rows
    r = np.arange(T * tr)
    ch = (r // tr) * half + (r % half)
    src = np.where((r % tr) < half, ch, I + ch)
    rows = torch.zeros(T * tr, K, dtype=torch.bfloat16)
    ok = torch.from_numpy(ch < I)
    rows[ok] = w[torch.from_numpy(src[ch < I])]
    assert torch.equal(wp.data.cpu().view(torch.int16), _pack_reference(rows, tr))


def test_add_rmsnorm_splitk(cuda):
    g = torch.Generator().manual_seed(42)
    M, N, S = 40, 2048, 3
    part = torch.randn(S, M, N, generator=g)
    h = torch.randn(M, N, generator=g).bfloat16()
    gamma = (torch.rand(N, generator=g) + 0.5).bfloat16()
    hd = h.to(cuda)
    out = _ops().add_rmsnorm_splitk(hd, part.to(cuda).reshape(-1), S, gamma.to(cuda), 1e-6)
    torch.cuda.synchronize()
    o = O.rnd(part.double().sum(0), torch.bfloat16)
    h_ref = O.rnd(h.double() + o, torch.bfloat16)
    assert torch.equal(hd.cpu().double(), h_ref)
    assert _maxdiff(out, O.rmsnorm(h_ref, gamma, 1e-6)) <= BF16_ATOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_embedding_rmsnorm_equals_two_calls(cuda, dtype):
    """The decode step's fused gather + first RMSNorm equals ll_embedding then
    ll_rmsnorm bit for bit (int64 and int32 ids, repeated ids)."""
    ops = _ops()
    g = torch.Generator().manual_seed(44)
    table = torch.randn(1000, 2048, generator=g).to(dtype).to(cuda)
    gamma = (torch.rand(2048, generator=g) + 0.5).to(dtype).to(cuda)
    for ids in (torch.randint(0, 1000, (40,), generator=g),
                torch.tensor([7, 7, 999, 0], dtype=torch.int32)):
        ids = ids.to(cuda)
        h, x = ops.embedding_rmsnorm(table, ids, gamma, 1e-6)
        h2 = ops.embedding(table, ids)
        x2 = ops.rmsnorm(h2, gamma, 1e-6)
        torch.cuda.synchronize()
        assert torch.equal(h, h2) and torch.equal(x, x2)


def test_silu_and_mul_splitk(cuda):
    g = torch.Generator().manual_seed(43)
    M, N, S = 40, 1376, 2
    part = torch.randn(S, M, 2 * N, generator=g)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    _ops().silu_and_mul_splitk(part.to(cuda).reshape(-1), S, out)
    torch.cuda.synchronize()
    gu = O.rnd(part.double().sum(0), torch.bfloat16)
    assert _close_rel(out, O.silu_and_mul(gu, torch.bfloat16))


@pytest.mark.parametrize("dtype,cs", [(torch.bfloat16, torch.float32), (torch.float16, torch.float16)])
def test_rope_kv_scatter_vec_equals_scalar(cuda, dtype, cs):
    """The 4-pairs-per-thread path (head_dim % 8 == 0, aligned rows) against the
    one-pair path (forced by a row stride that is not a multiple of 4) on the
    same inputs: q rows and pool bit-identical."""
    g = torch.Generator().manual_seed(24)
    T, H, KVH, D, P = 37, 16, 2, 128, 100
    W = (H + 2 * KVH) * D
    qkv = torch.randn(T, W, generator=g).to(dtype)
    pos = torch.randint(0, 300, (T,), generator=g)
    cos, sin = O.rope_table(320, D)
    cos, sin = cos.to(cs).to(cuda), sin.to(cs).to(cuda)
    slots = torch.from_numpy(np.random.RandomState(5).permutation(P)[:T].astype(np.int32)).to(cuda)
    a = qkv.to(cuda)
    wide = torch.zeros(T, W + 2, dtype=dtype)
    wide[:, :W] = qkv
    b = wide.to(cuda)[:, :W]  # row stride W + 2: the scalar path
    pa = torch.zeros(P, 2 * KVH, D, dtype=dtype, device=cuda)
    pb = torch.zeros_like(pa)
    _ops().rope_kv_scatter(a, H, KVH, D, pos.to(cuda), cos, sin, slots, pa)
    _ops().rope_kv_scatter(b, H, KVH, D, pos.to(cuda), cos, sin, slots, pb)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(pa, pb)


def test_rope_kv_scatter_splitk(cuda):
    g = torch.Generator().manual_seed(44)
    T, H, KVH, D, P, S = 40, 16, 2, 128, 100, 4
    W_ = (H + 2 * KVH) * D
    part = torch.randn(S, T, W_, generator=g) * 0.5
    bias = (torch.randn(W_, generator=g) * 0.1).bfloat16()
    pos = torch.randint(0, 1200, (T,), generator=g).int()
    cos, sin = O.rope_table(1300, D)
    slots = torch.from_numpy(np.random.RandomState(4).permutation(P)[:T].astype(np.int32))
    pool = torch.zeros(P, 2 * KVH, D, dtype=torch.bfloat16, device=cuda)
    q = torch.empty(T, H * D, dtype=torch.bfloat16, device=cuda)
    _ops().rope_kv_scatter_splitk(part.to(cuda).reshape(-1), S, bias.to(cuda), q, H, KVH, D,
                                  pos.to(cuda), cos.float().to(cuda), sin.float().to(cuda),
                                  slots.to(cuda), pool)
    torch.cuda.synchronize()
    qkv = O.rnd(part.double().sum(0) + bias.double(), torch.bfloat16)
    c, s_ = cos[pos.long()], sin[pos.long()]
    q_ref = O.rotary(qkv[:, :H * D].view(T, H, D), c, s_)
    k_ref = O.rotary(qkv[:, H * D:(H + KVH) * D].view(T, KVH, D), c, s_)
    # the partials are summed in fp32 (oracle: fp64), which can move a bf16
    # rounding of qkv by one ulp before the rotation
    assert _maxdiff(q.view(T, H, D), q_ref) <= BF16_ATOL
    assert _maxdiff(pool[slots.long(), :KVH], k_ref) <= BF16_ATOL
    assert torch.equal(pool[slots.long(), KVH:].cpu().double(), qkv[:, (H + KVH) * D:].view(T, KVH, D))


# ------------------------------------------------------------ slot table
def test_assign_slots(cuda):
    """ll_assign_slots: req_to_tokens[rows, cols] = slots (the table update of
    PageCache.alloc_token_idxs, cache.py:238-248), over three rounds that
    overwrite earlier entries."""
    ops = _ops()
    g = torch.Generator().manual_seed(41)
    n = 40
    ref = torch.zeros(50, 700, dtype=torch.int32)
    r2t = ref.clone().to(cuda)
    for _ in range(3):
        rows = torch.randperm(50, generator=g)[:n].to(torch.int32)
        cols = torch.randint(0, 700, (n,), generator=g, dtype=torch.int32)
        slots = torch.randint(0, 1 << 20, (n,), generator=g, dtype=torch.int32)
        ref[rows.long(), cols.long()] = slots
        ops.assign_slots(r2t, torch.stack([slots, rows, cols]).to(cuda), n)
    torch.cuda.synchronize()
    assert torch.equal(r2t.cpu(), ref)


@pytest.mark.parametrize("M,N,K,dtype", [
    (40, 151936, 2048, torch.bfloat16),  # the 3B lm_head: one split, 128-row tiles
    (1, 151936, 2048, torch.bfloat16),
    (64, 151936, 2048, torch.float16),
    (17, 1024, 256, torch.bfloat16),     # tiny vocabulary: one split, 64-row tiles
    (40, 2048, 2048, torch.bfloat16),    # a plan with k splits: GEMM, then ll_argmax
])
def test_gemm_packed_argmax_equals_gemm_then_argmax(cuda, M, N, K, dtype):
    """ll_gemm_packed_f32_argmax (the argmax's first pass in the lm_head
    epilogue) against ll_gemm_packed_f32 followed by ll_argmax on the same
    inputs: fp32 logits bit-identical, tokens identical. Rows 0 and 1 of the
    weight are copied to the last rows and to a row in the middle (other
    tiles), and token row 0 of x is scaled so those rows win: exact ties
    across tiles, where the first index must win. With a set status word
    every token is -1."""
    ops = _ops()
    g = torch.Generator().manual_seed(M + N + K)
    w = (torch.randn(N, K, generator=g) * 0.05).to(dtype)
    w[N - 1] = w[0]
    w[N // 2 + 3] = w[0]
    w[N - 2] = w[1]
    x = torch.randn(M, K, generator=g).to(dtype)
    x[0] = (w[0].float() * 4).to(dtype)  # row 0 of w (and its copies) is the maximum for token 0
    print(f"case: gemm_packed_argmax M={M} N={N} K={K} {dtype}", flush=True)
    xd, wp = x.to(cuda), ops.PackedWeight(w.to(cuda))
    ref_logits = ops.gemm_packed(xd, wp, out_dtype=torch.float32)
    ref_tok = ops.argmax(ref_logits)
    logits, tok = ops.gemm_packed_argmax(xd, wp)
    torch.cuda.synchronize()
    assert torch.equal(logits, ref_logits)
    assert torch.equal(tok, ref_tok)
    assert int(tok[0]) == 0  # the first of the tied copies
    status = torch.ones(1, dtype=torch.int32, device=cuda)
    _, tok_err = ops.gemm_packed_argmax(xd, wp, status=status)
    assert torch.equal(tok_err.cpu(), torch.full((M,), -1, dtype=torch.int64))
    status.zero_()
    _, tok_ok = ops.gemm_packed_argmax(xd, wp, status=status)
    assert torch.equal(tok_ok, ref_tok)
