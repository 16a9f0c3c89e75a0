"""Pins of the oracle's generation driver (CPU only).

* A shared prefix prefilled once and reused by prompt-cache prefills gives the
  same greedy tokens and logits as prefilling every full prompt: the identity
  the radix cache relies on (flash_attn_v2.py:699-762 vs :513-566), here at
  the whole-model level, float and W8A8.
* Teacher forcing with the oracle's own tokens reproduces its free-running
  generation.
* float32 arithmetic (used for the full-width geometries) stays within
  rounding of the float64 oracle.
"""
import torch

from oracle import ops
from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle
from tests.model_weights import moving_state_dict


def _tiny(hidden=256, inter=688):
    from lite_lang_amd.models.qwen2.weights import Qwen2Config
    c = Qwen2Config(layer_nums=2, hidden_size=hidden, num_heads=4, num_key_value_heads=2,
                    intermediate_size=inter, vocab_size=1024)
    oc = Qwen2Cfg(num_layers=2, hidden=hidden, heads=4, kv_heads=2, intermediate=inter, vocab=1024)
    return c, oc


def _prompts(seed):
    g = torch.Generator().manual_seed(seed)
    prefix = torch.randint(0, 1024, (24,), generator=g).tolist()
    prompts = [prefix + torch.randint(0, 1024, (n,), generator=g).tolist() for n in (3, 9, 1)]
    prompts.insert(1, torch.randint(0, 1024, (30,), generator=g).tolist())  # no shared prefix
    return prefix, prompts


def test_shared_prefix_equals_full_prefill():
    for quant, inter in ((None, 688), ("w8a8", 768)):
        cfg, ocfg = _tiny(inter=inter)
        sd = moving_state_dict(cfg, seed=21)
        prefix, prompts = _prompts(21)
        full, lf = Qwen2Oracle(ocfg, sd, torch.float32, 8, 64, 512, quant=quant).generate(
            prompts, 6, return_logits=True)
        shared, ls = Qwen2Oracle(ocfg, sd, torch.float32, 8, 64, 512, quant=quant).generate(
            prompts, 6, return_logits=True, prefix=prefix)
        assert torch.equal(full, shared), quant
        assert float((lf - ls).abs().max()) < 1e-5, quant
        assert len({tuple(t) for t in full.tolist()}) == 4


def test_teacher_forcing_with_own_tokens_is_free_running():
    cfg, ocfg = _tiny()
    sd = moving_state_dict(cfg, seed=22)
    _, prompts = _prompts(22)
    free, lf = Qwen2Oracle(ocfg, sd, torch.bfloat16, 8, 64, 512).generate(
        prompts, 8, return_logits=True)
    forced, lt = Qwen2Oracle(ocfg, sd, torch.bfloat16, 8, 64, 512).generate(
        prompts, 8, return_logits=True, feed=free)
    assert torch.equal(free, forced) and torch.equal(lf, lt)
    # feeding other tokens changes the later steps
    other = (free + 1) % 1024
    moved = Qwen2Oracle(ocfg, sd, torch.bfloat16, 8, 64, 512).generate(prompts, 8, feed=other)
    assert torch.equal(moved[:, 0], free[:, 0]) and not torch.equal(moved, free)


def test_fp32_math_within_rounding_of_fp64():
    cfg, ocfg = _tiny()
    sd = moving_state_dict(cfg, seed=23)
    _, prompts = _prompts(23)
    t64, l64 = Qwen2Oracle(ocfg, sd, torch.float32, 8, 64, 512).generate(
        prompts, 5, return_logits=True)
    with ops.math_dtype(torch.float32):
        t32, l32 = Qwen2Oracle(ocfg, sd, torch.float32, 8, 64, 512).generate(
            prompts, 5, return_logits=True, feed=t64)
    assert l32.dtype == torch.float32
    assert float((l64 - l32.double()).abs().max()) < 1e-4
