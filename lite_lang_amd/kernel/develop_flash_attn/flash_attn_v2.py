"""NoPad varlen prefill attention over the paged KV pool, drop-in for
litelang/kernel/develop_flash_attn/flash_attn_v2.py:513-566 and :699-762.

The other names the reference module exports (triton_attention,
gqa_context_attention, standard_attention_no_pad, standard_softmax_attention)
are imported by the reference model (transformer_layer.py:12-18) but never
called on its token loop; they exist here for import compatibility only and
raise if called.
"""
import torch

from lite_lang_amd import ops


@torch.no_grad()
def context_attention_fwd_with_no_pad_and_kv_cache(
    q, k, v, o, b_req_idx, b_start_loc, b_seq_len, max_input_len, req_to_token_indexs
):
    """Causal attention of the NoPad query rows of each request over the first
    b_seq_len[b] slots of its slot-table row; writes o."""
    Lq, Lk, Lv = q.shape[-1], k.shape[-1], v.shape[-1]
    assert Lq == Lk and Lk == Lv
    assert Lk in {16, 32, 64, 128, 256}
    ops.prefill_attention(q, k, v, o, b_req_idx, b_start_loc, b_seq_len, int(max_input_len),
                          req_to_token_indexs)


@torch.no_grad()
def context_attention_fwd_with_no_pad_and_kv_cache_and_prompt_cache(
    q,
    k,
    v,
    o,
    b_req_idx,
    b_start_loc,
    b_seq_len,
    b_shared_seq_len,
    max_input_len,
    req_to_token_indexs,
):
    """As above, with the first b_shared_seq_len[b] keys of each request already
    cached (radix prefix hit): q holds only the b_seq_len - shared new rows."""
    Lq, Lk, Lv = q.shape[-1], k.shape[-1], v.shape[-1]
    assert Lq == Lk and Lk == Lv
    assert Lk in {16, 32, 64, 128, 256}
    ops.prefill_attention(q, k, v, o, b_req_idx, b_start_loc, b_seq_len, int(max_input_len),
                          req_to_token_indexs, b_shared_seq_len=b_shared_seq_len)


def _unused(name):
    def fn(*args, **kwargs):
        raise NotImplementedError(
            f"{name} is not part of the lite_lang token loop; use "
            "context_attention_fwd_with_no_pad_and_kv_cache")
    fn.__name__ = name
    return fn


triton_attention = _unused("triton_attention")
gqa_context_attention = _unused("gqa_context_attention")
standard_attention_no_pad = _unused("standard_attention_no_pad")
standard_softmax_attention = _unused("standard_softmax_attention")
