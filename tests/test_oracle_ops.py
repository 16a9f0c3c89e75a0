"""Pins of the CPU oracle's kernel restatements (oracle/ops.py).

Every check is independent of the oracle's own formula: a library routine
(torch.nn.functional), a closed form or special case, an invariant, or a
golden vector from the reference's files. Plausible mistakes (wrong eps
placement, swapped rotation sign, wrong GQA head map, off-by-one causal mask,
missing prompt-cache offset) each fail at least one test below.
"""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def test_rmsnorm_matches_library_and_closed_form():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(7, 96, generator=g, dtype=torch.float64) * 0.5 + 0.3
    gamma = torch.randn(96, generator=g, dtype=torch.float64)
    ref = F.rms_norm(x, (96,), gamma, eps=1e-5)
    torch.testing.assert_close(ops.rmsnorm(x, gamma, 1e-5), ref, rtol=1e-12, atol=1e-12)
    # constant row c with gamma=1: c / sqrt(c^2 + eps)
    c = torch.full((1, 64), -3.0, dtype=torch.float64)
    out = ops.rmsnorm(c, torch.ones(64, dtype=torch.float64), 1e-6)
    assert torch.allclose(out, torch.full_like(c, -3.0 / math.sqrt(9.0 + 1e-6)), atol=1e-15)


def test_rope_invariants():
    T, H, D = 9, 3, 32
    g = torch.Generator().manual_seed(2)
    x = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    cos, sin = ops.rope_table(64, D, 1e6, table_dtype=torch.float64)
    pos = torch.arange(T)
    y = ops.rotary(x, cos[pos], sin[pos])
    # position 0 is the identity
    torch.testing.assert_close(y[0], x[0])
    # each (i, i + D/2) pair keeps its norm
    n0 = x[..., : D // 2] ** 2 + x[..., D // 2:] ** 2
    n1 = y[..., : D // 2] ** 2 + y[..., D // 2:] ** 2
    torch.testing.assert_close(n0, n1)
    # relative position: <R(p)q, R(p')k> depends on p - p' only
    q = torch.randn(1, 1, D, generator=g, dtype=torch.float64)
    k = torch.randn(1, 1, D, generator=g, dtype=torch.float64)
    def dot(pq, pk):
        a = ops.rotary(q, cos[pq:pq + 1], sin[pq:pq + 1])
        b = ops.rotary(k, cos[pk:pk + 1], sin[pk:pk + 1])
        return float((a * b).sum())
    assert abs(dot(5, 2) - dot(13, 10)) < 1e-5  # table built in fp32 (pre_layer.py:23-26)
    # rotation direction: x0' = x0 cos - x1 sin (a sign flip fails here)
    e = torch.zeros(1, 1, D, dtype=torch.float64)
    e[0, 0, 0] = 1.0
    c1, s1 = torch.tensor([[0.6] * (D // 2)], dtype=torch.float64), torch.tensor([[0.8] * (D // 2)], dtype=torch.float64)
    r = ops.rotary(e, c1, s1)
    assert r[0, 0, 0] == pytest.approx(0.6) and r[0, 0, D // 2] == pytest.approx(0.8)


def test_rope_table_matches_pre_layer_formula():
    cos, sin = ops.rope_table(16, 8, 1e6)
    assert cos.dtype == torch.float16
    # theta^(-2i/D) with i=1, D=8 at p=3: cos(3 * 1e6^-0.25)
    assert float(cos[3, 1]) == pytest.approx(math.cos(3 * 1e6 ** -0.25), abs=1e-3)
    assert float(sin[0, 2]) == 0.0 and float(cos[0, 3]) == 1.0


def test_silu_and_mul_matches_library():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 40, generator=g, dtype=torch.float64)
    ref = F.silu(x[:, :20]) * x[:, 20:]
    torch.testing.assert_close(ops.silu_and_mul(x, torch.float64), ref)
    # fp16 rounding of silu happens before the multiply
    r16 = ops.silu_and_mul(x, torch.float16)
    exp = F.silu(x[:, :20]).to(torch.float16).to(torch.float64) * x[:, 20:]
    torch.testing.assert_close(r16, exp)


def _sdpa_decode(q, k_rows, v_rows, scale):
    return F.scaled_dot_product_attention(q[None, None], k_rows[None, None], v_rows[None, None],
                                          scale=scale)[0, 0]


def test_decode_attention_vs_sdpa_gqa_and_slots():
    g = torch.Generator().manual_seed(4)
    B, H, KVH, D, P = 3, 6, 2, 16, 50
    q = torch.randn(B, H, D, generator=g, dtype=torch.float64)
    kp = torch.randn(P, KVH, D, generator=g, dtype=torch.float64)
    vp = torch.randn(P, KVH, D, generator=g, dtype=torch.float64)
    r2t = torch.from_numpy(np.random.RandomState(0).permutation(P)[:40].reshape(4, 10).astype(np.int32))
    rids = [2, 0, 3]
    lens = [10, 1, 7]
    out = ops.decode_attention(q, r2t, rids, lens, kp, vp)
    for b in range(B):
        sl = r2t[rids[b], :lens[b]].long()
        for h in range(H):
            kv = h // (H // KVH)
            ref = _sdpa_decode(q[b, h:h + 1], kp[sl, kv], vp[sl, kv], 1 / math.sqrt(D))
            torch.testing.assert_close(out[b, h], ref[0])
    # len 1 gives the V row itself
    torch.testing.assert_close(out[1, 4], vp[r2t[0, 0].long(), 1])


def test_decode_attention_slot_permutation_invariance():
    g = torch.Generator().manual_seed(5)
    B, H, KVH, D, P = 2, 4, 1, 8, 20
    q = torch.randn(B, H, D, generator=g, dtype=torch.float64)
    kp = torch.randn(P, KVH, D, generator=g, dtype=torch.float64)
    vp = torch.randn(P, KVH, D, generator=g, dtype=torch.float64)
    r2t = torch.arange(P, dtype=torch.int32).view(2, 10)
    perm = torch.from_numpy(np.random.RandomState(1).permutation(P))
    inv = torch.argsort(perm)
    a = ops.decode_attention(q, r2t, [0, 1], [10, 6], kp, vp)
    b = ops.decode_attention(q, inv[r2t.long()].to(torch.int32), [0, 1], [10, 6], kp[perm], vp[perm])
    torch.testing.assert_close(a, b)


def test_prefill_attention_vs_sdpa_causal():
    g = torch.Generator().manual_seed(6)
    H, KVH, D, P = 4, 2, 16, 64
    lens = [5, 9]
    starts = [0, 5]
    T = sum(lens)
    q = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    kp = torch.randn(P, KVH, D, generator=g, dtype=torch.float64)
    vp = torch.randn(P, KVH, D, generator=g, dtype=torch.float64)
    r2t = torch.from_numpy(np.random.RandomState(2).permutation(P)[:32].reshape(2, 16).astype(np.int32))
    out = ops.prefill_attention(q, kp, vp, [1, 0], starts, lens, r2t)
    for b, rid in enumerate([1, 0]):
        sl = r2t[rid, :lens[b]].long()
        for h in range(H):
            kv = h // 2
            ref = F.scaled_dot_product_attention(
                q[starts[b]:starts[b] + lens[b], h][None], kp[sl, kv][None], vp[sl, kv][None],
                is_causal=True, scale=1 / math.sqrt(D))[0]
            torch.testing.assert_close(out[starts[b]:starts[b] + lens[b], h], ref)


def test_prompt_cache_equals_suffix_of_full_prefill():
    g = torch.Generator().manual_seed(7)
    H, KVH, D, P = 2, 1, 8, 40
    L, S = 12, 5
    q_full = torch.randn(L, H, D, generator=g, dtype=torch.float64)
    kp = torch.randn(P, KVH, D, generator=g, dtype=torch.float64)
    vp = torch.randn(P, KVH, D, generator=g, dtype=torch.float64)
    r2t = torch.arange(P, dtype=torch.int32).view(2, 20)
    full = ops.prefill_attention(q_full, kp, vp, [1], [0], [L], r2t)
    part = ops.prefill_attention(q_full[S:], kp, vp, [1], [0], [L], r2t, b_shared_seq_len=[S])
    torch.testing.assert_close(part, full[S:])


def test_online_softmax_kat():
    kat = json.load(open(os.path.join(GOLD, "softmax_kat.json")))
    x = torch.tensor(kat["x"], dtype=torch.float64)
    # a single query whose scores are x (q = x, K = identity rows, V = identity)
    q = x.view(1, 1, 3)
    kp = torch.eye(3, dtype=torch.float64).view(3, 1, 3)
    out = ops.decode_attention(q, torch.tensor([[0, 1, 2]], dtype=torch.int32), [0], [3], kp, kp,
                               sm_scale=1.0)
    torch.testing.assert_close(out[0, 0], torch.tensor(kat["softmax"], dtype=torch.float64))


def test_linear_and_argmax():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(3, 12, generator=g, dtype=torch.float64)
    w = torch.randn(5, 12, generator=g, dtype=torch.float64)
    b = torch.randn(5, generator=g, dtype=torch.float64)
    torch.testing.assert_close(ops.linear(x, w, b), F.linear(x, w, b))
    t = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0], [0.0, -1.0, 7.0, 7.0]])
    assert ops.argmax_first(t).tolist() == [1, 0, 2]


def test_w8a8_quantisation_closed_forms():
    w = torch.tensor([[0.5, -1.0, 0.25, 0.0], [2.0, 1.0, -0.0078125, 0.0]])
    q, s = ops.quantize_weight_per_channel_absmax(w)
    assert s.tolist() == pytest.approx([1.0 / 127, 2.0 / 127])
    # 0.5 * 127 = 63.5 -> 64 (half to even), -127, 31.75 -> 32, 0
    assert q[0].tolist() == [64, -127, 32, 0]
    # row 1: 127, 63.5 -> 64, -0.496 -> 0
    assert q[1].tolist() == [127, 64, 0, 0]
    g = torch.Generator().manual_seed(9)
    xq = torch.randint(-128, 128, (4, 64), generator=g, dtype=torch.int8)
    wq = torch.randint(-128, 128, (6, 64), generator=g, dtype=torch.int8)
    acc = ops.int8_gemm_i32(xq, wq)
    brute = [[sum(int(xq[t, k]) * int(wq[o, k]) for k in range(64)) for o in range(6)] for t in range(4)]
    assert acc.tolist() == brute


def test_oracle_weight_quantiser_pinned():
    """quantize_weight_per_channel_absmax against what the formula fixes
    (smooth_quant/layer.py:5-16): the scale is dtype(absmax / 127); the
    largest-magnitude entry maps to +-127; every code is within half a step of
    w / s; exact halves round to even; an all-zero row gives zero codes."""
    import torch
    from oracle.ops import quantize_weight_per_channel_absmax
    g = torch.Generator().manual_seed(70)
    w = (torch.randn(8, 64, generator=g) * 0.03).bfloat16()
    w[2] = 0
    # row 3: scale exactly 1/127 * 127 -> s = 1 when absmax = 127 (bf16-exact);
    # entries 2.5 and 3.5 are exact halves: round to 2 and 4
    w[3] = 0
    w[3, 0], w[3, 1], w[3, 2], w[3, 3] = 127.0, 2.5, 3.5, -0.5
    q, s = quantize_weight_per_channel_absmax(w)
    assert s.dtype == torch.bfloat16
    assert torch.equal(s, (w.abs().max(dim=1)[0].float() / 127).bfloat16())
    assert q[3, :4].tolist() == [127, 2, 4, 0]
    assert torch.equal(q[2], torch.zeros(64, dtype=torch.int8))
    wf, sf = w.float(), s.float().view(-1, 1)
    for r in (0, 1, 4, 5, 6, 7):
        assert int(q[r].abs().max()) == 127
        err = (q[r].float() * sf[r] - wf[r]).abs()
        assert float(err.max()) <= float(sf[r]) / 2 + 1e-7


def test_oracle_token_quantiser_pinned():
    """quantize_per_token_absmax against hand-computed codes: s_t =
    max_k |x[t, k]| / 127 in fp32; codes round half to even; the row's
    largest magnitude codes to +-127; an all-zero row gets scale 1 and codes
    0; no code can fall below -127 (|x| <= absmax, so |x / s| <= 127 up to
    one rounding), so the -128 clamp only matters for a static scale, whose
    clamping is pinned here too. Inputs arrive in the model dtype (bf16 and
    fp16 hold every value below exactly)."""
    from oracle.ops import quantize_per_token_absmax, quantize_static
    rows = [
        [127.0, 63.5, -0.5, 1.5, 2.5, -127.0, 0.25, -63.5],   # s = 1
        [0.0] * 8,                                             # s = 1 by definition
        [-254.0, 5.0, -3.0, 1.0, 127.0, 0.0, 3.0, -1.0],       # s = 2
        [0.75, -0.375, 0.1875, 0.0, 0.0, 0.0, 0.0, -0.09375],  # s = 0.75 / 127
    ]
    want = [
        [127, 64, 0, 2, 2, -127, 0, -64],
        [0] * 8,
        [-127, 2, -2, 0, 64, 0, 2, 0],
        # 0.375 * 127 / 0.75 = 63.5 -> 64 (even); 0.1875 -> 31.75 -> 32;
        # 0.09375 -> 15.875 -> 16
        [127, -64, 32, 0, 0, 0, 0, -16],
    ]
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        q, s = quantize_per_token_absmax(torch.tensor(rows, dtype=dt))
        assert q.dtype == torch.int8 and s.dtype == torch.float32
        assert q.tolist() == want, dt
        assert s[:3].tolist() == [1.0, 1.0, 2.0]
        assert float(s[3]) == float(torch.tensor(0.75, dtype=torch.float32) / 127)
    # random rows: the absmax entry codes to +-127 and every code is within
    # half a step of x / s (no code is clamped)
    g = torch.Generator().manual_seed(71)
    x = (torch.randn(16, 96, generator=g) * torch.rand(16, 1, generator=g) * 3).bfloat16()
    q, s = quantize_per_token_absmax(x)
    xd, sd = x.double(), s.double()
    for r in range(16):
        assert int(q[r].abs().max()) == 127 and int(q[r].min()) >= -127
        # exact error of the code; the fp32 division x / s may move a value
        # by 127 * 2^-24 of a step across the half-way point
        err = (q[r].double() * sd[r] - xd[r]).abs()
        assert float(err.max()) <= float(sd[r]) * (0.5 + 1e-5)
    # static scale: the clamp at both ends, ties to even
    qs, ss = quantize_static(torch.tensor([[-1000.0, 1000.0, 2.5, -2.5, 127.5, -128.5]]), 1.0)
    assert qs.tolist() == [[-128, 127, 2, -2, 127, -128]] and ss.tolist() == [1.0]


def test_oracle_dequant_pinned():
    """dequant_int32 = (fp32(acc) * s_tok[m]) * fp32(s_ch[n]) on hand-computed
    exact cases, including the fp32 conversion of an int32 sum above 2^24
    (16777217 rounds to even, 16777216) and 16-bit channel scales."""
    from oracle.ops import dequant_int32
    acc = torch.tensor([[100, -7], [0, 1 << 20], [16777217, 16777219]], dtype=torch.int32)
    s_tok = torch.tensor([0.5, 2.0 ** -10, 1.0], dtype=torch.float32)
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        s_ch = torch.tensor([0.25, 3.0], dtype=dt)
        y = dequant_int32(acc, s_tok, s_ch)
        assert y.dtype == torch.float32
        assert y.tolist() == [[12.5, -10.5], [0.0, 3072.0], [4194304.0, 50331660.0]]
