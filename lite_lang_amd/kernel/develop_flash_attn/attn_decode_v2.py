"""Import-compatibility module for litelang/kernel/develop_flash_attn/attn_decode_v2.py.

The reference model imports decode_flash_attention, gqa_decode_attention_fwd
and gqa_reference_impl (transformer_layer.py:4-8) but decodes with
token_decode_attention_flash_decoding; these names raise if called.
"""


def _unused(name):
    def fn(*args, **kwargs):
        raise NotImplementedError(
            f"{name} is not part of the lite_lang token loop; use "
            "token_decode_attention_flash_decoding")
    fn.__name__ = name
    return fn


decode_flash_attention = _unused("decode_flash_attention")
gqa_decode_attention_fwd = _unused("gqa_decode_attention_fwd")
gqa_reference_impl = _unused("gqa_reference_impl")
standard_softmax_attention = _unused("standard_softmax_attention")
