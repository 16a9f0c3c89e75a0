"""Rotary embedding, drop-in for litelang/kernel/develop_rope/rope.py:154-198."""
import torch

from lite_lang_amd import ops


@torch.no_grad()
def rotary_emb_fwd(q, k, cos, sin):
    """In-place rotate-half RoPE on q [T, Hq, D] and k [T, Hk, D] (k may be a
    strided view into the KV pool) with per-token cos/sin [T, D/2]."""
    assert q.shape[0] == cos.shape[0] and q.shape[0] == sin.shape[0], (
        f"q shape {q.shape} cos shape {cos.shape}")
    assert k.shape[0] == cos.shape[0] and k.shape[0] == sin.shape[0], (
        f"k shape {k.shape} cos shape {cos.shape}")
    if cos.stride(-1) != 1:
        cos = cos.contiguous()
    if sin.stride(-1) != 1:
        sin = sin.contiguous()
    ops.rotary_emb(q, k, cos, sin)
    return
