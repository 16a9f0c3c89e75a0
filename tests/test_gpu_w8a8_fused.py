"""W8A8 consumers that dequantise int32 partials inline, against
ll_dequant_splitk followed by the fp32 consumer on the same partials: every
output bit-identical (the inline dequantisation is the same fp32 arithmetic
in the same order), including add+RMSNorm's per-token int8 output against
ll_quant_per_token on its stored row, and the fused RoPE attention's output
and pool. The fused quantisation of the attention output for the o_proj
(per token and static) equals the separate quantiser on the stored rows. Scale dtypes fp32 / fp16 / bf16, several split counts, the
attention with several splits (quantised in the merge) and with one."""
import numpy as np
import pytest
import torch

from oracle import ops as O

pytestmark = pytest.mark.gpu


def _ops():
    from lite_lang_amd import ops
    return ops


def _parts(g, S, M, N, sdt, cuda):
    part = torch.randint(-30000, 30000, (S, M, N), generator=g, dtype=torch.int32)
    st = torch.rand(M, generator=g) * 1e-3 + 1e-5
    sc = (torch.rand(N, generator=g) * 1e-2 + 1e-4).to(sdt)
    ops = _ops()
    return ops.I8Partials(part.to(cuda).reshape(-1), S, st.to(cuda), sc.to(cuda))


def _dequant(p, M, N, cuda):
    out = torch.empty(M, N, device=cuda)
    _ops().dequant_splitk(p.part, p.splits, p.s_tok, p.s_ch, out, M, N)
    return out


@pytest.mark.parametrize("S,N,sdt", [(3, 2048, torch.bfloat16), (1, 1536, torch.float16),
                                     (8, 2048, torch.float32), (5, 3584, torch.bfloat16)])
def test_add_rmsnorm_i32_with_quant(cuda, S, N, sdt):
    g = torch.Generator().manual_seed(70 + S)
    M = 40
    print(f"case: add_rmsnorm_i32 S={S} N={N} {sdt}", flush=True)
    ops = _ops()
    p = _parts(g, S, M, N, sdt, cuda)
    h0 = torch.randn(M, N, generator=g).bfloat16().to(cuda)
    gamma = (torch.rand(N, generator=g) + 0.5).bfloat16().to(cuda)
    ha, hb = h0.clone(), h0.clone()
    outa, qa, sa = ops.add_rmsnorm_splitk_i32(ha, p, gamma, 1e-6, quant=True)
    f = _dequant(p, M, N, cuda)
    outb = ops.add_rmsnorm_splitk(hb, f.reshape(-1), 1, gamma, 1e-6)
    qb, sb = ops.quant_per_token(outb)
    torch.cuda.synchronize()
    assert torch.equal(ha, hb) and torch.equal(outa, outb)
    assert torch.equal(qa, qb) and torch.equal(sa, sb)
    # the no-quant form writes the same h and output
    hc = h0.clone()
    outc = ops.add_rmsnorm_splitk_i32(hc, p, gamma, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(hc, hb) and torch.equal(outc, outb)


@pytest.mark.parametrize("S,N,sdt", [(1, 1376, torch.float16), (4, 11008, torch.bfloat16)])
def test_silu_and_mul_i32(cuda, S, N, sdt):
    g = torch.Generator().manual_seed(80 + S)
    M = 40
    print(f"case: silu_and_mul_i32 S={S} N={N}", flush=True)
    ops = _ops()
    p = _parts(g, S, M, 2 * N, sdt, cuda)
    a = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    b = torch.empty_like(a)
    ops.silu_and_mul_splitk_i32(p, a)
    f = _dequant(p, M, 2 * N, cuda)
    ops.silu_and_mul_splitk(f.reshape(-1), 1, b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("S,H,KVH,D,sdt", [(4, 16, 2, 128, torch.bfloat16),
                                           (1, 14, 2, 64, torch.float16)])
def test_rope_attention_i32(cuda, S, H, KVH, D, sdt):
    g = torch.Generator().manual_seed(90 + S)
    B = 6
    lens = [1, 17, 300, 64, 5, 129]
    cap = max(lens)
    W = (H + 2 * KVH) * D
    dt = torch.bfloat16 if sdt == torch.bfloat16 else torch.float16
    print(f"case: rope attention i32 S={S} H={H} KVH={KVH} D={D}", flush=True)
    ops = _ops()
    p = _parts(g, S, B, W, sdt, cuda)
    bias = (torch.randn(W, generator=g) * 0.1).to(dt).to(cuda)
    P = B * cap + 3
    pool = torch.randn(P, 2 * KVH, D, generator=g).to(dt).to(cuda)
    perm = torch.from_numpy(np.random.RandomState(S).permutation(P)[: B * cap].astype(np.int32))
    r2t = perm.view(B, cap).to(cuda)
    slots = torch.tensor([int(r2t[b, l - 1]) for b, l in enumerate(lens)], dtype=torch.int32,
                         device=cuda)
    pos = torch.tensor([l - 1 for l in lens], dtype=torch.int32, device=cuda)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=cuda)
    rids = torch.arange(B, dtype=torch.int32, device=cuda)
    cos, sin = O.rope_table(cap + 8, D)
    cos, sin = cos.float().to(cuda), sin.float().to(cuda)
    pa, pb = pool.clone(), pool.clone()
    oa = torch.empty(B, H, D, dtype=dt, device=cuda)
    ob = torch.empty_like(oa)
    ops.decode_attention_rope_splitk_i32(p, bias, pos, cos, sin, slots, r2t, rids, lens_t, cap,
                                         pa[:, :KVH], pa[:, KVH:], oa)
    f = _dequant(p, B, W, cuda)
    ops.decode_attention_rope_splitk(f.reshape(-1), 1, bias, pos, cos, sin, slots, r2t, rids,
                                     lens_t, cap, pb[:, :KVH], pb[:, KVH:], ob)
    torch.cuda.synchronize()
    assert torch.equal(pa, pb) and torch.equal(oa, ob)


_LENS40 = np.random.RandomState(7).randint(1, 700, size=40).tolist()


@pytest.mark.parametrize("lens,static", [([1, 17, 300, 64, 5, 129], False),
                                         ([1, 17, 300, 64, 5, 129], True),
                                         ([3, 9, 12, 1, 20, 7], False),
                                         (_LENS40, False),
                                         (_LENS40, True)])
def test_rope_attention_i32_quant(cuda, lens, static):
    """The quantising variant (split merge of every head of a sequence in the
    split stage when the sequence is split, else a separate quantiser) against
    the plain variant followed by the quantiser: bit-identical rows, pool,
    codes and scales. 40 ragged sequences put 5 sequences on every XCD."""
    g = torch.Generator().manual_seed(95)
    S, H, KVH, D, B = 4, 16, 2, 128, len(lens)
    cap = max(lens)
    W = (H + 2 * KVH) * D
    ops = _ops()
    from lite_lang_amd import _lib
    nsplit_gt1 = _lib.load().ll_decode_attention_workspace_size(B, H, KVH, D, cap) > 0
    print(f"case: rope attention i32 quant static={static} several splits={nsplit_gt1}",
          flush=True)
    p = _parts(g, S, B, W, torch.bfloat16, cuda)
    bias = (torch.randn(W, generator=g) * 0.1).bfloat16().to(cuda)
    P = B * cap + 3
    pool = torch.randn(P, 2 * KVH, D, generator=g).bfloat16().to(cuda)
    perm = torch.from_numpy(np.random.RandomState(4).permutation(P)[: B * cap].astype(np.int32))
    r2t = perm.view(B, cap).to(cuda)
    slots = torch.tensor([int(r2t[b, l - 1]) for b, l in enumerate(lens)], dtype=torch.int32,
                         device=cuda)
    pos = torch.tensor([l - 1 for l in lens], dtype=torch.int32, device=cuda)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=cuda)
    rids = torch.arange(B, dtype=torch.int32, device=cuda)
    cos, sin = O.rope_table(cap + 8, D)
    cos, sin = cos.float().to(cuda), sin.float().to(cuda)
    sa = torch.tensor([0.021], device=cuda) if static else None
    pa, pb = pool.clone(), pool.clone()
    oa = torch.empty(B, H, D, dtype=torch.bfloat16, device=cuda)
    ob = torch.empty_like(oa)
    _, qa, sqa = ops.decode_attention_rope_splitk_i32(
        p, bias, pos, cos, sin, slots, r2t, rids, lens_t, cap, pa[:, :KVH], pa[:, KVH:], oa,
        quant=True, input_scale=sa)
    ops.decode_attention_rope_splitk_i32(p, bias, pos, cos, sin, slots, r2t, rids, lens_t, cap,
                                         pb[:, :KVH], pb[:, KVH:], ob)
    flat = ob.view(B, H * D)
    qb, sqb = ops.quant_static(flat, sa) if static else ops.quant_per_token(flat)
    torch.cuda.synchronize()
    assert torch.equal(oa, ob) and torch.equal(pa, pb)
    assert torch.equal(qa, qb) and torch.equal(sqa, sqb)


@pytest.mark.parametrize("M,I,K,sdt,odt", [(40, 11008, 2048, torch.bfloat16, torch.bfloat16),
                                           (1, 1376, 512, torch.float16, torch.float16),
                                           (17, 8960, 1536, torch.float32, torch.bfloat16),
                                           (64, 1000, 256, torch.bfloat16, torch.bfloat16)])
def test_i8_gate_up_silu_fused(cuda, M, I, K, sdt, odt):
    """The int8 gate/up GEMM with dequantisation and SiLU_and_Mul in its
    epilogue against the int32 partials of the plain int8 GEMM followed by
    silu_and_mul_splitk_i32: bit-identical (the int32 sums are exact whatever
    the split, and both sides dequantise and round in the same order). I=11008
    takes 128-row tiles, the others 64-row ones; I=1000 ends in a partial tile."""
    g = torch.Generator().manual_seed(100 + M)
    print(f"case: i8 gate/up silu M={M} I={I} K={K} {sdt} -> {odt}", flush=True)
    ops = _ops()
    wq = torch.randint(-127, 128, (2 * I, K), generator=g, dtype=torch.int8).to(cuda)
    sc = (torch.rand(2 * I, generator=g) * 2e-3 + 1e-4).to(sdt).to(cuda)
    xq = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8).to(cuda)
    st = (torch.rand(M, generator=g) * 1e-2 + 1e-4).to(cuda)
    pg = ops.PackedI8GateUp(wq, sc)
    a = torch.empty(M, I, dtype=odt, device=cuda)
    ops.gemm_i8_gate_up_silu(xq, st, pg, a)
    pw = ops.PackedI8Weight(wq, sc)
    s = ops.gemm_i8_splitk_count(M, 2 * I, K)
    part = torch.empty(s * M * 2 * I, dtype=torch.int32, device=cuda)
    ops.gemm_i8_splitk_packed(xq, pw, part)
    b = torch.empty_like(a)
    ops.silu_and_mul_splitk_i32(ops.I8Partials(part, s, st, sc), b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # the products are not degenerate: some outputs are far from zero
    assert float(a.float().abs().max()) > 1.0
