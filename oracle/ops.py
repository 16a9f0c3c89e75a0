"""CPU restatement of the hot-path ops (test infrastructure only).

All arithmetic is float64 unless a function says otherwise; ``rnd`` emulates
storing an intermediate in a low-precision dtype, at the points where the
reference stores one. Reference paths are relative to the lite_lang root.

``math_dtype(torch.float32)`` switches the float arithmetic to fp32 inside a
``with`` block. It is used only where float64 would take minutes on the CPU
(the full-width Qwen2 geometries and the CPU baseline); every pin in
tests/test_oracle_*.py runs in float64. The integer paths (quantisers, int8
GEMM) are exact in either mode.
"""
from __future__ import annotations

import contextlib
import math

import numpy as np
import torch


_MATH = [torch.float64]


def compute_dtype() -> torch.dtype:
    """The float type the oracle computes in (float64 unless math_dtype is active)."""
    return _MATH[-1]


@contextlib.contextmanager
def math_dtype(dt: torch.dtype):
    """Compute in `dt` (float32 or float64) inside the block."""
    assert dt in (torch.float32, torch.float64)
    _MATH.append(dt)
    try:
        yield
    finally:
        _MATH.pop()


def rnd(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Round x to `dtype` storage (RNE) and come back to the compute dtype."""
    return x.to(dtype).to(compute_dtype())


# ---------------------------------------------------------------- RMSNorm
def rmsnorm(x: torch.Tensor, gamma: torch.Tensor, eps: float) -> torch.Tensor:
    """(x / sqrt(sum(x^2)/N + eps)) * gamma.

    Follows torch_rmsnorm, litelang/kernel/develop_rmsnorm/rms_norm.py:11-17
    (the kernel, rms_norm.py:37-53, does the same in fp32 and casts at the end).
    """
    x = x.to(compute_dtype())
    var = (x * x).sum(-1, keepdim=True) / x.shape[-1]
    return x / torch.sqrt(var + eps) * gamma.to(compute_dtype())


# ---------------------------------------------------------------- RoPE
def rope_table(max_length: int, head_dim: int, theta: float = 1e6,
               table_dtype: torch.dtype = torch.float16):
    """cos/sin[p, i] = cos/sin(p * theta^(-2i/D)), built in fp32 and stored in
    fp16, as Qwen2PreLayer._ComputePosition (pre_layer.py:21-30)."""
    freqs = 1.0 / theta ** (torch.arange(0, head_dim, 2) / head_dim)
    pos = torch.arange(0, max_length)
    ang = pos[:, None] * freqs[None, :]
    return torch.cos(ang).to(table_dtype), torch.sin(ang).to(table_dtype)


def rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of x [T, H, D] with per-token cos/sin [T, D/2].

    Follows torch_rotary_emb, litelang/kernel/develop_rope/rope.py:225-234.
    """
    x = x.to(compute_dtype())
    T, H, D = x.shape
    x0, x1 = x[..., : D // 2], x[..., D // 2:]
    c = cos.to(compute_dtype()).view(T, 1, D // 2)
    s = sin.to(compute_dtype()).view(T, 1, D // 2)
    return torch.cat((x0 * c - x1 * s, x0 * s + x1 * c), dim=-1)


# ---------------------------------------------------------------- SiLU_and_Mul
def silu_and_mul(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """up * dtype(silu(gate)) with gate = x[:, :N], up = x[:, N:].

    Follows silu_and_mul.py:80-84 plus the kernel's rounding of silu before
    the multiply (silu_and_mul.py:43-50; the reference rounds to fp16, its
    only runtime dtype; here to the model dtype).
    """
    x = x.to(compute_dtype())
    n = x.shape[-1] // 2
    g, u = x[:, :n], x[:, n:]
    s = rnd(g / (1.0 + torch.exp(-g)), dtype)
    return u * s


# ---------------------------------------------------------------- attention
def decode_attention(q, req_to_tokens, b_req_idx, b_seq_len, k_pool, v_pool, sm_scale=None):
    """out[b, h] = softmax(q . K[slots]^T * scale) . V[slots] over the first
    b_seq_len[b] slots of row b_req_idx[b]; KV head = h // (H / KVH).

    Follows the per-head loop of test_flash_decoding
    (flash_decoding.py:348-366) with the slot gather of stage 1
    (flash_decoding.py:74-88); float64 softmax. k_pool / v_pool are [P, KVH, D].
    """
    B, H, D = q.shape
    KVH = k_pool.shape[1]
    G = H // KVH
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    out = torch.zeros((B, H, D), dtype=compute_dtype())
    for b in range(B):
        L = int(b_seq_len[b])
        if L <= 0:
            continue
        slots = req_to_tokens[int(b_req_idx[b]), :L].long()
        for kv in range(KVH):
            k = k_pool[slots, kv].to(compute_dtype())
            v = v_pool[slots, kv].to(compute_dtype())
            for h in range(kv * G, (kv + 1) * G):
                s = (q[b, h].to(compute_dtype()) @ k.T) * sm_scale
                out[b, h] = torch.softmax(s, -1) @ v
    return out


def prefill_attention(q, k_pool, v_pool, b_req_idx, b_start_loc, b_seq_len, req_to_tokens,
                      b_shared_seq_len=None, sm_scale=None, p_dtype=None):
    """Causal NoPad prefill over the slot table.

    For request b with L keys and S shared: query rows start+m, m < L-S,
    attend to keys n <= m + S. Follows the masked per-head reference of
    flash_attn_v2.py:826-855 / 934-964, with the prompt-cache offset of
    flash_attn_v2.py:660-662. If p_dtype is given the probabilities are
    rounded to it before P.V and the normaliser uses the unrounded values,
    as the kernel does (flash_attn_v2.py:488-499).
    """
    T, H, D = q.shape
    KVH = k_pool.shape[1]
    G = H // KVH
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    out = torch.zeros((T, H, D), dtype=compute_dtype())
    for b in range(len(b_seq_len)):
        L = int(b_seq_len[b])
        S = int(b_shared_seq_len[b]) if b_shared_seq_len is not None else 0
        st = int(b_start_loc[b])
        nq = L - S
        if nq <= 0:
            continue
        slots = req_to_tokens[int(b_req_idx[b]), :L].long()
        m = torch.arange(nq)[:, None] + S
        n = torch.arange(L)[None, :]
        mask = n <= m
        for h in range(H):
            kv = h // G
            if h % G == 0:
                k = k_pool[slots, kv].to(compute_dtype())
                v = v_pool[slots, kv].to(compute_dtype())
            s = (q[st:st + nq, h].to(compute_dtype()) @ k.T) * sm_scale
            s = torch.where(mask, s, torch.tensor(-math.inf, dtype=compute_dtype()))
            mx = s.max(-1, keepdim=True).values
            p = torch.exp(s - mx)
            l = p.sum(-1, keepdim=True)
            if p_dtype is not None:
                p = rnd(p, p_dtype)
            out[st:st + nq, h] = (p @ v) / l
    return out


# ---------------------------------------------------------------- dense
def linear(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """x [M, K] . w[N, K]^T (+ bias), float64 accumulation.

    The reference computes torch.addmm / torch.mm with pre-transposed weights
    (transformer_layer.py:80,82,95-109,193); the product is the same matrix
    product. Third-party arithmetic (cuBLAS) -- pinned by the closed form
    only.
    """
    y = x.to(compute_dtype()) @ w.to(compute_dtype()).T
    if bias is not None:
        y = y + bias.to(compute_dtype())
    return y


def argmax_first(x: torch.Tensor) -> torch.Tensor:
    """Index of the first maximum of each row (torch.argmax tie rule used by
    Qwen2PostLayer._PostProcess, post_layer.py:75-77)."""
    a = x.detach().cpu().numpy()
    return torch.from_numpy(np.argmax(a, axis=-1).astype(np.int64))


# ---------------------------------------------------------------- W8A8
def quantize_weight_per_channel_absmax(w: torch.Tensor):
    """s_o = max_i |w[o, i]| / 127 in w's dtype; w_q = clamp(round_half_even(
    fp32(w) / fp32(s_o)), -128, 127).

    Follows quantize/smooth_quant/layer.py:5-16 on its CPU path: the scale is
    computed in the weight's dtype (:8), then the weight is taken to fp32 (:11)
    and divided by the promoted scale (:13); torch.round is round-half-to-even.
    An all-zero row (0/0) is defined here as q = 0. Returns (int8 [N, K],
    scales [N] in w's dtype).
    """
    s = w.abs().max(dim=1)[0] / 127
    q = w.to(torch.float32) / s.to(torch.float32).view(-1, 1)
    q = torch.nan_to_num(q, nan=0.0).round().clamp(-128, 127).to(torch.int8)
    return q, s


def quantize_per_token_absmax(x: torch.Tensor):
    """Dynamic per-token activation quantisation: s_t = max_k |x[t, k]| / 127
    in fp32 (1 for an all-zero row), x_q = clamp(round_half_even(fp32(x) /
    s_t), -128, 127). The rule is build-defined: the reference has no runtime
    activation quantisation, and smooth_quant/layer.py:5-16 fixes only the
    weight side, whose absmax / 127 rule this mirrors per token. Pinned by
    hand-computed codes (ties to even, the absmax entry at +-127, the zero
    row) in tests/test_oracle_ops.py."""
    x = x.to(torch.float32)
    s = x.abs().max(dim=1)[0] / 127
    s = torch.where(s > 0, s, torch.ones_like(s))
    q = (x / s.view(-1, 1)).round().clamp(-128, 127).to(torch.int8)
    return q, s


def int8_gemm_i32(xq: torch.Tensor, wq: torch.Tensor) -> torch.Tensor:
    """Exact int32 accumulators acc[t, o] = sum_k xq[t, k] * wq[o, k].

    Evaluated as a float64 matrix product, which is exact here: every product
    and every partial sum is an integer of magnitude <= 128 * 128 * K, below
    2^53 for any K < 2^39, so no float64 operation rounds (and the int32
    result holds for K <= 131071)."""
    assert xq.shape[-1] < (1 << 17)
    return (xq.to(torch.float64) @ wq.to(torch.float64).T).to(torch.int64).to(torch.int32)


def quantize_static(x: torch.Tensor, s_a):
    """Static per-tensor activation quantisation with a calibrated input scale
    (the quant_scale buffer of smooth_quant/layer.py:63-94; the reference has
    no runtime that applies it, so the rule is build-defined and the same as
    the per-token one with a fixed scale): s = fp32(s_a);
    q = clamp(round_half_even(fp32(x) / s), -128, 127). Returns (q, s_tok [M]
    all equal to s)."""
    s = float(s_a)
    q = (x.to(torch.float32) / torch.tensor(s, dtype=torch.float32)).round().clamp(-128, 127)
    return q.to(torch.int8), torch.full((x.shape[0],), s, dtype=torch.float32)


def dequant_int32(acc: torch.Tensor, s_tok: torch.Tensor, s_ch: torch.Tensor) -> torch.Tensor:
    """fp32(acc) * s_tok[m] * fp32(s_ch[n]), evaluated in fp32 in that order
    (build-defined dequantisation of the W8A8 runtime)."""
    return (acc.to(torch.float32) * s_tok.to(torch.float32).view(-1, 1)) * s_ch.to(torch.float32).view(1, -1)
