"""Qwen2 configuration and weights.

Qwen2Config mirrors litelang/models/qwen2/model.py:7-21 (it reads the same
config.json keys and derives head_dim = hidden / heads). Weights arrive as a
Hugging Face style state dict -- from safetensors files (the loader of
model.py:61-97) or from `random_state_dict` for the random-init benchmark
configurations -- and are packed once into the device layout:

  embed      [V, hidden]
  wqkv       [(H + 2*KVH) * D, hidden]   rows: q heads, k heads, v heads
  bqkv       [(H + 2*KVH) * D]
  wo         [hidden, H * D]             (o_proj bias is ignored, as the
                                          reference does: transformer_layer.py:193)
  wgu        [2 * I, hidden]             rows: gate then up
  wgu_il     [2 * I, hidden]             the same rows in 64-row blocks that
                                         alternate gate and up (the prefill
                                         gate/up + SiLU tile kernel's layout)
  wdown      [hidden, I]
  ln1, ln2   [hidden]
  norm       [hidden]
  lm_head    [V, hidden]                 (= embed when tied)

All matrices keep the nn.Linear [out, in] layout (the reference transposes to
[in, out] for torch.mm, load_weights.py:22-28); the GEMM kernels stream both
operands k-contiguous.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

import torch


@dataclass
class Qwen2Config:
    layer_nums: int
    hidden_size: int
    num_heads: int
    num_key_value_heads: int
    intermediate_size: int
    vocab_size: int
    tie_word_embeddings: bool = True
    rms_norm_eps: float = 1e-6
    final_norm_eps: float = 1e-5   # post_layer.py:12
    rope_theta: float = 1e6        # pre_layer.py:22

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads  # model.py:19

    @classmethod
    def from_json(cls, config_path: str) -> "Qwen2Config":
        with open(config_path, "r", encoding="utf-8") as f:
            c = json.load(f)
        return cls(layer_nums=c["num_hidden_layers"], hidden_size=c["hidden_size"],
                   num_heads=c["num_attention_heads"],
                   num_key_value_heads=c["num_key_value_heads"],
                   intermediate_size=c["intermediate_size"], vocab_size=c["vocab_size"],
                   tie_word_embeddings=c.get("tie_word_embeddings", True))

    def num_params(self) -> int:
        D, H, KVH, hd, I, V = (self.head_dim, self.num_heads, self.num_key_value_heads,
                               self.hidden_size, self.intermediate_size, self.vocab_size)
        per_layer = (H + 2 * KVH) * D * hd + (H + 2 * KVH) * D + hd * H * D + 3 * I * hd + 2 * hd
        return self.layer_nums * per_layer + V * hd * (1 if self.tie_word_embeddings else 2) + hd


# The BASELINE configurations
def tiny_config() -> Qwen2Config:
    return Qwen2Config(layer_nums=2, hidden_size=256, num_heads=4, num_key_value_heads=2,
                       intermediate_size=688, vocab_size=1024)


def qwen2_1p5b_config() -> Qwen2Config:
    return Qwen2Config(layer_nums=28, hidden_size=1536, num_heads=12, num_key_value_heads=2,
                       intermediate_size=8960, vocab_size=151936)


def qwen25_3b_config() -> Qwen2Config:
    return Qwen2Config(layer_nums=36, hidden_size=2048, num_heads=16, num_key_value_heads=2,
                       intermediate_size=11008, vocab_size=151936)


def state_dict_shapes(cfg: Qwen2Config):
    """(name, shape, kind) in the canonical generation order; kind is 'w'
    (N(0, std)) or 'norm' (ones)."""
    D, H, KVH, hd, I, V = (cfg.head_dim, cfg.num_heads, cfg.num_key_value_heads,
                           cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size)
    out = [("model.embed_tokens.weight", (V, hd), "w")]
    for i in range(cfg.layer_nums):
        p = f"model.layers.{i}."
        out += [
            (p + "self_attn.q_proj.weight", (H * D, hd), "w"),
            (p + "self_attn.q_proj.bias", (H * D,), "w"),
            (p + "self_attn.k_proj.weight", (KVH * D, hd), "w"),
            (p + "self_attn.k_proj.bias", (KVH * D,), "w"),
            (p + "self_attn.v_proj.weight", (KVH * D, hd), "w"),
            (p + "self_attn.v_proj.bias", (KVH * D,), "w"),
            (p + "self_attn.o_proj.weight", (hd, H * D), "w"),
            (p + "mlp.gate_proj.weight", (I, hd), "w"),
            (p + "mlp.up_proj.weight", (I, hd), "w"),
            (p + "mlp.down_proj.weight", (hd, I), "w"),
            (p + "input_layernorm.weight", (hd,), "norm"),
            (p + "post_attention_layernorm.weight", (hd,), "norm"),
        ]
    out.append(("model.norm.weight", (hd,), "norm"))
    if not cfg.tie_word_embeddings:
        out.append(("lm_head.weight", (V, hd), "w"))
    return out


def random_state_dict(cfg: Qwen2Config, seed: int = 0, std: float = 0.02, device="cpu",
                      dtype=torch.float32):
    """Random-init weights: linear/embedding weights and q/k/v biases drawn
    N(0, std) from one torch.Generator seeded `seed`, in the order of
    state_dict_shapes; RMSNorm gammas = 1 (the Hugging Face init)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    sd = {}
    for name, shape, kind in state_dict_shapes(cfg):
        if kind == "norm":
            sd[name] = torch.ones(shape, device=device, dtype=dtype)
        else:
            t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
            sd[name] = (t * std).to(dtype)
    return sd


def load_state_dict(model_path: str):
    """Read every tensor of a (possibly sharded) checkpoint on the CPU
    (model.py:61-97): safetensors files, or the pytorch_model*.bin files the
    SmoothQuant converter writes (save_pretrained(..., safe_serialization=
    False), quantize/smooth_quant.py:245), read with torch.load(weights_only=
    True) so nothing in them is executed."""
    def shards(index_name):
        with open(os.path.join(model_path, index_name)) as f:
            return sorted(set(json.load(f)["weight_map"].values()))

    def exists(name):
        return os.path.exists(os.path.join(model_path, name))

    if exists("model.safetensors.index.json"):
        files = shards("model.safetensors.index.json")
    elif exists("model.safetensors"):
        files = ["model.safetensors"]
    elif exists("pytorch_model.bin.index.json"):
        files = shards("pytorch_model.bin.index.json")
    elif exists("pytorch_model.bin"):
        files = ["pytorch_model.bin"]
    else:
        raise FileNotFoundError(f"no model.safetensors or pytorch_model.bin in {model_path}")
    sd = {}
    for fn in files:
        path = os.path.join(model_path, fn)
        if fn.endswith(".safetensors"):
            from safetensors import safe_open
            with safe_open(path, framework="pt") as f:
                for k in f.keys():
                    sd[k] = f.get_tensor(k)
        else:
            sd.update(torch.load(path, map_location="cpu", weights_only=True))
    return sd


def is_int8_checkpoint(sd: dict) -> bool:
    """True for the SmoothQuant converter's output: int8 projection weights
    with per-channel weight_scale (quantize/smooth_quant/layer.py:19-94)."""
    w = sd.get("model.layers.0.self_attn.q_proj.weight")
    return w is not None and w.dtype == torch.int8


def check_smoothquant_config(model_path: str) -> None:
    """Reject converter settings this runtime cannot serve. With "qkv" or
    "fc1" set to "per-channel" the converter divides input_layernorm /
    post_attention_layernorm by the calibrated input scale
    (smooth_quant/qwen2.py:183-192) but stores that scale nowhere, so the
    int8 products of q/k/v (gate/up) could not be scaled back."""
    path = os.path.join(model_path, "quant_config.json")
    if not os.path.exists(path):
        return
    with open(path, encoding="utf-8") as f:
        qc = json.load(f)
    for key, norm in (("qkv", "input_layernorm"), ("fc1", "post_attention_layernorm")):
        if qc.get(key) == "per-channel":
            raise ValueError(
                f"quant_config {key!r} = 'per-channel': the converter folded the calibrated "
                f"input scale into {norm} without saving it, so these int8 outputs cannot be "
                "dequantised; convert with per-token activations for this projection")


class DeviceWeights:
    """Packed device copy of a state dict (layout in the module docstring)."""

    def __init__(self, cfg: Qwen2Config, sd: dict, dtype: torch.dtype, device, pack: bool = True,
                 quant: str = None):
        def dev(t):
            return t.to(device=device, dtype=dtype).contiguous()

        self.embed = dev(sd["model.embed_tokens.weight"])
        self.norm = dev(sd["model.norm.weight"])
        self.lm_head = self.embed if cfg.tie_word_embeddings else dev(sd["lm_head.weight"])
        int8 = is_int8_checkpoint(sd)
        if int8 and quant != "w8a8":
            raise ValueError("an int8 (SmoothQuant converter) checkpoint runs with quant='w8a8'")
        self.layers = []
        for i in range(cfg.layer_nums):
            p = f"model.layers.{i}."
            lw = {}
            if int8:  # the projections exist only as int8 (below)
                lw["wqkv"] = lw["wo"] = lw["wgu"] = lw["wdown"] = None
            else:
                lw["wqkv"] = dev(torch.cat([sd[p + "self_attn.q_proj.weight"],
                                            sd[p + "self_attn.k_proj.weight"],
                                            sd[p + "self_attn.v_proj.weight"]], 0))
                lw["wo"] = dev(sd[p + "self_attn.o_proj.weight"])
                lw["wgu"] = dev(torch.cat([sd[p + "mlp.gate_proj.weight"],
                                           sd[p + "mlp.up_proj.weight"]], 0))
                lw["wdown"] = dev(sd[p + "mlp.down_proj.weight"])
            bq = sd.get(p + "self_attn.q_proj.bias")
            lw["bqkv"] = None if bq is None else dev(torch.cat([
                bq, sd[p + "self_attn.k_proj.bias"], sd[p + "self_attn.v_proj.bias"]], 0))
            lw["ln1"] = dev(sd[p + "input_layernorm.weight"])
            lw["ln2"] = dev(sd[p + "post_attention_layernorm.weight"])
            self.layers.append(lw)
        # Decode-path projections also held in the weight-streaming kernel's
        # packed layout (one more copy of those weights; prefill keeps using
        # the [N, K] tensors). None where the layout does not apply.
        self.packed = [{} for _ in self.layers]
        self.lm_head_p = None
        self.quant = quant
        if quant == "w8a8":
            # int8 projections (per-channel scales), the lm_head stays in the
            # model dtype as in the reference (smooth_quant/qwen2.py:249-250)
            from lite_lang_amd import ops
            for i, (lw, pk) in enumerate(zip(self.layers, self.packed)):
                if int8:
                    for name, parts in _I8_GROUPS:
                        pk[name + "_i8"] = _int8_group(sd, f"model.layers.{i}.", parts, device)
                    continue
                for name in ("wqkv", "wo", "wgu", "wdown"):
                    pk[name + "_i8"] = ops.QuantWeight(lw[name], gate_up=(name == "wgu"))
            if pack and dtype in (torch.bfloat16, torch.float16):
                self.lm_head_p = ops.pack_weight(self.lm_head)
        elif pack and dtype in (torch.bfloat16, torch.float16) and torch.device(device).type == "cuda":
            from lite_lang_amd import ops
            for lw, pk in zip(self.layers, self.packed):
                for name in ("wqkv", "wo", "wdown"):
                    pk[name] = ops.pack_weight(lw[name])
                pk["wgu_silu"] = ops.pack_gate_up(lw["wgu"])
                # the prefill gate/up + SiLU tile kernel's interleaved copy
                K = lw["wgu"].shape[1]
                if ops.gemm_tiled_supported(65, lw["wgu"].shape[0], K, dtype):
                    lw["wgu_il"] = ops.interleave_gate_up(lw["wgu"])
            self.lm_head_p = ops.pack_weight(self.lm_head)

    def nbytes_streamed_per_decode(self) -> int:
        """Weight bytes one decode forward reads (embedding rows excluded)."""
        es = self.embed.element_size()
        n = (self.norm.numel() + self.lm_head.numel()) * es
        for lw, pk in zip(self.layers, self.packed):
            for name, v in lw.items():
                if name == "wgu_il":  # prefill-only copy
                    continue
                qw = pk.get(name + "_i8")
                if qw is not None:
                    n += qw.q.numel() + qw.scale.numel() * qw.scale.element_size()
                elif v is not None:
                    n += v.numel() * es
        return n


# int8 projection groups of a converted checkpoint: (runtime name, checkpoint
# modules concatenated along the output rows)
_I8_GROUPS = (("wqkv", ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")),
              ("wo", ("self_attn.o_proj",)),
              ("wgu", ("mlp.gate_proj", "mlp.up_proj")),
              ("wdown", ("mlp.down_proj",)))


def _int8_group(sd, prefix, parts, device):
    """QuantWeight of the converter's modules (W8A8BFP32OFP32Linear[WithQuantScale],
    smooth_quant/layer.py:19-94): int8 `weight` [out, in], `weight_scale` [out, 1]
    kept in its stored dtype, `quant_scale` (static input scale) when present."""
    from lite_lang_amd import ops
    q = torch.cat([sd[prefix + m + ".weight"] for m in parts], 0)
    s = torch.cat([sd[prefix + m + ".weight_scale"].reshape(-1) for m in parts], 0)
    a = [sd.get(prefix + m + ".quant_scale") for m in parts]
    if any(x is not None for x in a):
        if any(x is None for x in a) or len({float(x) for x in a}) != 1:
            raise ValueError(f"{prefix}{parts}: fused projections need one static input scale")
        a = float(a[0])
    else:
        a = None
    return ops.QuantWeight.from_int8(q.to(device), s.to(device), a,
                                     gate_up=(parts[0] == "mlp.gate_proj"))
