"""FlashDecoding paged decode attention, drop-in for
litelang/kernel/develop_flash_attn/flash_decoding.py:262-312."""
import torch

from lite_lang_amd import ops


def token_decode_attention_flash_decoding(
    q,
    req_to_token_indexs,
    b_req_idx,
    b_seq_len,
    max_len_in_batch,
    q_head_num,
    head_dim,
    cache_k,
    cache_v,
    out=None,
    alloc_tensor_func=torch.empty,
):
    """out[b, h] = softmax(q[b, h] . K^T / sqrt(head_dim)) . V over the first
    b_seq_len[b] slots of req_to_token_indexs[b_req_idx[b]].

    The split-K partials live in a persistent device workspace owned by the
    library (the reference allocates them per call with alloc_tensor_func,
    flash_decoding.py:286-295); alloc_tensor_func is still used for `out`.
    """
    Lk = cache_k.shape[-1]
    assert q.shape[-1] == Lk or q.numel() == q.size(0) * q_head_num * head_dim
    assert Lk in {16, 32, 64, 128}
    batch_size = q.size(0)
    calcu_shape1 = (batch_size, q_head_num, head_dim)
    o_tensor = (
        alloc_tensor_func(q.shape, dtype=q.dtype, device=q.device) if out is None else out
    )
    ops.decode_attention(
        q.view(calcu_shape1),
        req_to_token_indexs,
        b_req_idx,
        b_seq_len,
        int(max_len_in_batch),
        cache_k,
        cache_v,
        o_tensor.view(calcu_shape1),
    )
    return o_tensor
