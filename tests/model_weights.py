"""Seeded random Qwen2 weights whose greedy tokens move (test helper).

With the Hugging Face init (every weight N(0, 0.02), norm gains 1) the
residual stream of a shallow random model is dominated by the token's own
embedding row, so the tied lm_head scores the input token far above all others
and greedy decoding repeats one token forever: a token-level comparison would
then pass even with a broken KV write. Here the projections are scaled by
1.25 / sqrt(fan_in), so each layer's output is O(1) per element, the
embedding by 0.3 / sqrt(hidden), so the logits stay within about 1.7 in
magnitude: there two faithful bf16 executions of the model (the oracle in
float64 and in float32 arithmetic) differ by at most one bf16 step of the
logits (1/128), well inside the 2e-2 bar, while the greedy tokens move;
q/k/v biases N(0, 0.1) and every RMSNorm gain
U(0.8, 1.2). All draws come from one torch.Generator in the order of
state_dict_shapes.
"""
from __future__ import annotations

import math

import torch


def moving_state_dict(cfg, seed: int = 0, dtype=torch.float32, proj_gain: float = 1.25):
    from lite_lang_amd.models.qwen2.weights import state_dict_shapes
    g = torch.Generator().manual_seed(seed)
    emb = 0.3 / math.sqrt(cfg.hidden_size)
    sd = {}
    for name, shape, kind in state_dict_shapes(cfg):
        if kind == "norm":
            t = torch.rand(shape, generator=g) * 0.4 + 0.8
        elif "embed_tokens" in name or name.startswith("lm_head"):
            t = torch.randn(shape, generator=g) * emb
        elif name.endswith("bias"):
            t = torch.randn(shape, generator=g) * 0.1
        else:
            t = torch.randn(shape, generator=g) * (proj_gain / math.sqrt(shape[1]))
        sd[name] = t.to(dtype)
    return sd
