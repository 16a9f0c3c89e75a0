"""A tiny Qwen2 checkpoint written by Hugging Face transformers itself (offline,
seeded random weights) together with a byte-level BPE Qwen2Tokenizer trained
offline on a seeded synthetic corpus, for tests that cross-check the weight
loader, the tokenizer wrapper, the CPU oracle and the GPU path against an
implementation independent of all three.

The HF config is set to what the reference hard-codes (RoPE theta 1e6,
RMSNorm eps 1e-6); HF applies that eps to the final norm too, where the
reference uses 1e-5 (post_layer.py:12), so comparisons set the final-norm eps
to HF's. Weights are seeded normals scaled so that greedy decoding moves
between tokens with clear top-1 margins; norm gains U(0.8, 1.2). Token id 0
is <|endoftext|> (eos and pad, as in Qwen2 checkpoints).
"""
from __future__ import annotations

import json
import random

import torch

VOCAB = 1024
EOS = 0
EMBED_STD, PROJ_STD, BIAS_STD = 0.3, 0.08, 0.1


def corpus(n=3000, seed=0):
    """Sentences of made-up words (seeded)."""
    rng = random.Random(seed)
    syl = ["ka", "lo", "mi", "ten", "ra", "su", "vo", "pel", "dan", "or", "is", "the", "an",
           "ing", "ed", "qu", "zo", "fi", "be", "nu"]
    words = ["".join(rng.choice(syl) for _ in range(rng.randint(1, 3))) for _ in range(400)]
    return [" ".join(rng.choice(words) for _ in range(rng.randint(5, 15)))
            + rng.choice([".", ",", "!", "?"]) for _ in range(n)]


def tiny_hf_config():
    from transformers import Qwen2Config
    return Qwen2Config(vocab_size=VOCAB, hidden_size=256, intermediate_size=688,
                       num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                       max_position_embeddings=512, rms_norm_eps=1e-6, rope_theta=1e6,
                       tie_word_embeddings=True, eos_token_id=EOS, pad_token_id=EOS,
                       bos_token_id=None)


def make_checkpoint(path: str, seed: int = 0):
    """Write model.safetensors, config.json and the tokenizer files to path;
    return the HF model (fp32, eval mode)."""
    from tokenizers import Tokenizer, models, pre_tokenizers, trainers
    from transformers import Qwen2ForCausalLM, Qwen2Tokenizer

    model = Qwen2ForCausalLM(tiny_hf_config()).eval()
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.copy_(torch.rand(p.shape, generator=g) * 0.4 + 0.8)
            elif "embed_tokens" in name:
                p.copy_(torch.randn(p.shape, generator=g) * EMBED_STD)
            elif name.endswith("bias"):
                p.copy_(torch.randn(p.shape, generator=g) * BIAS_STD)
            else:
                p.copy_(torch.randn(p.shape, generator=g) * PROJ_STD)
    model.save_pretrained(path)

    bpe = Tokenizer(models.BPE())
    bpe.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    trainer = trainers.BpeTrainer(vocab_size=1000, special_tokens=["<|endoftext|>"],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  show_progress=False)
    bpe.train_from_iterator(corpus(), trainer)
    merges = [tuple(m) for m in json.loads(bpe.to_str())["model"]["merges"]]
    tok = Qwen2Tokenizer(vocab=bpe.get_vocab(), merges=merges, unk_token=None,
                         eos_token="<|endoftext|>", pad_token="<|endoftext|>")
    assert tok.eos_token_id == EOS and len(tok) <= VOCAB
    tok.save_pretrained(path)
    return model


def hf_greedy(model, prompt_ids, n_new):
    """Greedy continuation of one prompt by the HF model, one full forward per
    step (no generate() machinery, no eos stop, first index on ties): (new ids
    [n_new], raw last-position logits [n_new, V])."""
    ids = list(prompt_ids)
    new, logits = [], []
    with torch.no_grad():
        for _ in range(n_new):
            lg = model(torch.tensor([ids]), use_cache=False).logits[0, -1].float()
            t = int(torch.argmax(lg))
            new.append(t)
            logits.append(lg)
            ids.append(t)
    return torch.tensor(new), torch.stack(logits, 0)


def min_margin(logits):
    """Smallest top-1 minus top-2 logit gap over the steps."""
    top2 = logits.topk(2, dim=-1).values
    return float((top2[:, 0] - top2[:, 1]).min())


PROJ = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
        "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def make_smoothquant_checkpoint(path: str, model, calib_ids, dtype=torch.float16,
                                quant_config=None):
    """Write what the reference's SmoothQuant converter saves
    (quantize/smooth_quant.py:225-245 via QuantizedQwen2ForCausalLM,
    smooth_quant/qwen2.py) for the float HF model, with smoothing factors of 1
    (smoothing re-balances float weights before quantisation and does not
    change the format):
      * every projection: int8 `weight` and `weight_scale` [out, 1] from
        quantize_weight_per_channel_absmax on the weight in `dtype`
        (smooth_quant/layer.py:5-16, restated in oracle/ops.py);
      * o_proj and down_proj: `quant_scale` = max |input| / 127 in `dtype`
        over the calibration prompts (collect_llama_layer_scales,
        quantize/smooth_quant.py:123-140);
      * q/k/v biases, norms and embeddings in `dtype`; lm_head tied (not
        stored); pytorch_model.bin (save_pretrained(safe_serialization=False)),
        config.json and quant_config.json."""
    import os
    from oracle.ops import quantize_weight_per_channel_absmax
    act = {}

    def hook(mod, inp, out, name):
        act[name] = max(act.get(name, 0.0), float(inp[0].abs().max()))

    hooks = [m.register_forward_hook(lambda mod, i, o, name=name: hook(mod, i, o, name))
             for name, m in model.named_modules()
             if name.endswith("self_attn.o_proj") or name.endswith("mlp.down_proj")]
    with torch.no_grad():
        for ids in calib_ids:
            model(torch.tensor([list(ids)]), use_cache=False)
    for h in hooks:
        h.remove()
    sd = {}
    for k, v in model.state_dict().items():
        if k == "lm_head.weight":
            continue
        mod = k.rsplit(".", 1)[0]
        if k.endswith(".weight") and mod.split("layers.")[-1].split(".", 1)[-1] in PROJ:
            q, s = quantize_weight_per_channel_absmax(v.to(dtype))
            sd[k] = q
            sd[mod + ".weight_scale"] = s.view(-1, 1)
            if mod in act:
                sd[mod + ".quant_scale"] = torch.tensor(act[mod] / 127, dtype=dtype)
        else:
            sd[k] = v.to(dtype)
    os.makedirs(path, exist_ok=True)
    torch.save(sd, os.path.join(path, "pytorch_model.bin"))
    model.config.save_pretrained(path)
    qc = quant_config or {"qkv": "per-token", "out": "per-tensor", "fc1": "per-token",
                          "fc2": "per-tensor"}
    with open(os.path.join(path, "quant_config.json"), "w", encoding="utf-8") as f:
        json.dump(qc, f)
    return sd
