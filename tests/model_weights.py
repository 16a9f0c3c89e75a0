"""Seeded random Qwen2 weights whose greedy tokens move (test helper).

With the Hugging Face init (every weight N(0, 0.02), norm gains 1) the
residual stream of a shallow random model is dominated by the token's own
embedding row, so the tied lm_head scores the input token far above all others
and greedy decoding repeats one token forever: a token-level comparison would
then pass even with a broken KV write. Here the projections are scaled by
1.25 / sqrt(fan_in), so each layer's output is O(1) per element, the
embedding by 0.65 / sqrt(hidden), so the logits stay below 4 in magnitude
(bf16 steps of at most 1/64 there, so one rounding flip stays under 2e-2),
q/k/v biases N(0, 0.1) and every RMSNorm gain
U(0.8, 1.2). All draws come from one torch.Generator in the order of
state_dict_shapes.
"""
from __future__ import annotations

import math

import torch


def moving_state_dict(cfg, seed: int = 0, dtype=torch.float32):
    from lite_lang_amd.models.qwen2.weights import state_dict_shapes
    g = torch.Generator().manual_seed(seed)
    emb = 0.65 / math.sqrt(cfg.hidden_size)
    sd = {}
    for name, shape, kind in state_dict_shapes(cfg):
        if kind == "norm":
            t = torch.rand(shape, generator=g) * 0.4 + 0.8
        elif "embed_tokens" in name or name.startswith("lm_head"):
            t = torch.randn(shape, generator=g) * emb
        elif name.endswith("bias"):
            t = torch.randn(shape, generator=g) * 0.1
        else:
            t = torch.randn(shape, generator=g) * (1.25 / math.sqrt(shape[1]))
        sd[name] = t.to(dtype)
    return sd
