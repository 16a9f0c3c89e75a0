"""Fused decode step of one layer's attention: ll_decode_attention_rope_splitk
(QKV split-K partials -> bias -> RoPE -> new token's K/V into the pool ->
paged GQA attention) against the two-call sequence ll_rope_kv_scatter_splitk +
ll_decode_attention on the same inputs.

The bar is bit-identity of the attention output AND of the whole pool: the
fused kernel restates the same arithmetic (partials summed in split order,
bias in fp32, rounding to the model dtype, the same rotation), and the split
geometry of the attention is the same. The two-call sequence is itself held
to the CPU oracle by test_gpu_ops.py; here the fused output is also checked
against the oracle directly (bf16/fp16 max-abs 2e-2), so a mistake shared by
both GPU paths would still fail.

Cases cover one and several attention splits, QKV split counts 1/3/4/6,
bias present or absent, bf16 and fp16, head_dim 64 and 128, GQA group sizes
1..16, lengths 1 (only the new token), 16 (full tile), 17 (new tile), long
sequences, a launch bound above every length, int32 and int64 index tensors.
"""
import numpy as np
import pytest
import torch

from oracle import ops as O

pytestmark = pytest.mark.gpu


def _ops():
    from lite_lang_amd import ops
    return ops


def _case(cuda, B, H, KVH, D, lens, S, dtype, seed, bias=True, max_len=None, rids=None,
          idx64=False):
    g = torch.Generator().manual_seed(seed)
    max_len = max_len or max(lens)
    cap = max(max_len, max(lens))
    W = (H + 2 * KVH) * D
    P = B * cap + 5
    part = torch.randn(S, B, W, generator=g) * 0.5
    bvec = (torch.randn(W, generator=g) * 0.1).to(dtype) if bias else None
    pool = torch.randn(P, 2 * KVH, D, generator=g).to(dtype)
    perm = np.random.RandomState(seed).permutation(P)[: B * cap].astype(np.int32)
    rids = rids if rids is not None else list(range(B))
    r2t = torch.zeros(max(rids) + 2, cap, dtype=torch.int32)
    for b, r in enumerate(rids):
        r2t[r] = torch.from_numpy(perm[b * cap:(b + 1) * cap])
    slots = torch.tensor([int(r2t[r, l - 1]) for r, l in zip(rids, lens)], dtype=torch.int32)
    # the decode-step precondition: a new slot is read by its own sequence only
    for b, (r, l) in enumerate(zip(rids, lens)):
        for b2, (r2, l2) in enumerate(zip(rids, lens)):
            if b2 != b:
                assert int(slots[b]) not in r2t[r2, :l2].tolist()
    pos = torch.tensor([l - 1 for l in lens])
    cos, sin = O.rope_table(cap + 8, D)
    it = torch.int64 if idx64 else torch.int32
    dev = dict(
        part=part.to(cuda).contiguous(), bias=bvec.to(cuda) if bias else None,
        pos=pos.to(it).to(cuda), cos=cos.float().to(cuda), sin=sin.float().to(cuda),
        slots=slots.to(cuda), r2t=r2t.to(cuda), rids=torch.tensor(rids, dtype=it, device=cuda),
        lens=torch.tensor(lens, dtype=it, device=cuda))
    return dev, pool, max_len, (part, bvec, pos, cos, sin, slots, r2t, rids)


def _two_call(cuda, d, pool, B, H, KVH, D, S, max_len, dtype):
    ops = _ops()
    pa = pool.to(cuda)
    q = torch.empty(B, H * D, dtype=dtype, device=cuda)
    out = torch.empty(B, H, D, dtype=dtype, device=cuda)
    ops.rope_kv_scatter_splitk(d["part"].reshape(-1), S, d["bias"], q, H, KVH, D, d["pos"],
                               d["cos"], d["sin"], d["slots"], pa)
    ops.decode_attention(q.view(B, H, D), d["r2t"], d["rids"], d["lens"], max_len,
                         pa[:, :KVH], pa[:, KVH:], out)
    return out, pa


def _fused(cuda, d, pool, B, H, KVH, D, S, max_len, dtype):
    ops = _ops()
    pb = pool.to(cuda)
    out = torch.empty(B, H, D, dtype=dtype, device=cuda)
    ops.decode_attention_rope_splitk(d["part"].reshape(-1), S, d["bias"], d["pos"], d["cos"],
                                     d["sin"], d["slots"], d["r2t"], d["rids"], d["lens"],
                                     max_len, pb[:, :KVH], pb[:, KVH:], out)
    return out, pb


def _oracle(host, pool, H, KVH, D, lens, dtype):
    part, bvec, pos, cos, sin, slots, r2t, rids = host
    qkv = part.double().sum(0)
    if bvec is not None:
        qkv = qkv + bvec.double()
    qkv = O.rnd(qkv, dtype)
    B = qkv.shape[0]
    q = qkv[:, : H * D].view(B, H, D)
    k = qkv[:, H * D:(H + KVH) * D].view(B, KVH, D)
    v = qkv[:, (H + KVH) * D:].view(B, KVH, D)
    c, s = cos[pos.long()], sin[pos.long()]
    q = O.rnd(O.rotary(q, c, s), dtype)
    k = O.rnd(O.rotary(k, c, s), dtype)
    pool = pool.clone()
    pool[slots.long(), :KVH] = k.to(dtype)
    pool[slots.long(), KVH:] = v.to(dtype)
    return O.decode_attention(q.to(dtype), r2t, rids, lens, pool[:, :KVH], pool[:, KVH:])


CASES = [
    # name, B, H, KVH, D, lens, S, dtype, bias, max_len
    ("config2-like", 40, 12, 2, 128, None, 4, torch.bfloat16, True, None),
    ("3b-heads", 3, 16, 2, 128, [1, 17, 2000], 6, torch.bfloat16, True, None),
    ("d64-fp16-nobias", 3, 14, 2, 64, [5, 100, 33], 1, torch.float16, False, None),
    ("g16", 4, 16, 1, 128, [16, 300, 64, 1], 3, torch.bfloat16, True, None),
    ("mha-d64", 5, 8, 8, 64, [2, 16, 31, 129, 700], 4, torch.float16, True, None),
    ("single-token", 1, 12, 2, 128, [1], 4, torch.bfloat16, True, None),
    ("bound-above-lengths", 6, 12, 2, 128, [3, 40, 90, 17, 1, 250], 4, torch.bfloat16, True,
     4096),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_equals_two_call(cuda, case):
    name, B, H, KVH, D, lens, S, dtype, bias, max_len = case
    if lens is None:
        lens = np.random.RandomState(7).randint(1, 601, size=B).tolist()
    print(f"case: fused rope+attention {name} B={B} H={H} KVH={KVH} D={D} S={S} {dtype}",
          flush=True)
    d, pool, ml, host = _case(cuda, B, H, KVH, D, lens, S, dtype, 11, bias, max_len,
                              rids=np.random.RandomState(B).permutation(B + 1)[:B].tolist())
    oa, pa = _two_call(cuda, d, pool, B, H, KVH, D, S, ml, dtype)
    ob, pb = _fused(cuda, d, pool, B, H, KVH, D, S, ml, dtype)
    torch.cuda.synchronize()
    assert torch.equal(pa, pb), "pool contents differ"
    assert torch.equal(oa, ob), f"attention output differs (max {float((oa.float() - ob.float()).abs().max())})"
    ref = _oracle(host, pool, H, KVH, D, lens, dtype)
    err = float((ob.cpu().double() - ref).abs().max())
    assert err <= 2e-2, f"fused output vs oracle max-abs {err}"


def test_fused_int64_indices_and_repeat(cuda):
    B, H, KVH, D, S = 4, 12, 2, 128, 4
    lens = [33, 1, 512, 48]
    print("case: fused rope+attention int64 indices, two calls", flush=True)
    d, pool, ml, host = _case(cuda, B, H, KVH, D, lens, S, torch.bfloat16, 3, idx64=True)
    oa, pa = _two_call(cuda, d, pool, B, H, KVH, D, S, ml, torch.bfloat16)
    ob, pb = _fused(cuda, d, pool, B, H, KVH, D, S, ml, torch.bfloat16)
    oc, pc = _fused(cuda, d, pool, B, H, KVH, D, S, ml, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(pa, pb) and torch.equal(pb, pc)
    assert torch.equal(oa, ob) and torch.equal(ob, oc)


def test_fused_rejects_unsupported(cuda):
    from lite_lang_amd import _lib
    ops = _ops()
    B, H, KVH, D, S = 2, 4, 2, 32, 1
    d, pool, ml, _ = _case(cuda, B, H, KVH, D, [4, 5], S, torch.bfloat16, 0)
    pb = pool.to(cuda)
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(_lib.LiteLangError, match="head_dim 64 or 128"):
        ops.decode_attention_rope_splitk(d["part"].reshape(-1), S, d["bias"], d["pos"], d["cos"],
                                         d["sin"], d["slots"], d["r2t"], d["rids"], d["lens"],
                                         ml, pb[:, :KVH], pb[:, KVH:], out)
