"""CPU restatement of the Qwen2 token loop (test infrastructure only).

Dataflow follows litelang/models/qwen2/model.py:48-59 (Qwen2Model.forward),
layer/pre_layer.py:15-30, layer/transformer_layer.py:46-194 and
layer/post_layer.py:14-77, with the reference quirks kept:
  * per-layer RMSNorm eps 1e-6 (transformer_layer.py:41), final norm eps 1e-5
    (post_layer.py:12);
  * RoPE theta 1e6, cos/sin table built in fp32 and stored fp16
    (pre_layer.py:21-30);
  * K rotated before it is written to the pool (transformer_layer.py:115,143);
  * o_proj bias ignored (transformer_layer.py:193);
  * residual adds stored in the model dtype (transformer_layer.py:69,76);
  * greedy argmax, first index on ties (post_layer.py:75-77), on the logits
    kept unrounded (fp32/fp64): the build writes fp32 logits and argmaxes
    those (the reference stores its fp16 ones).
Compute is float64 (fp32 inside ops.math_dtype(torch.float32), used for the
full-width geometries only); `rnd` stores an intermediate in the model dtype
wherever the reference stores a tensor.

Weights come in as a Hugging Face style state dict (the names read by
layer_weights/load_weights.py:86-172 and pre/post_layer_weights.py).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from .cache import PageCache
from .runner_batch import Req, no_padding_messages


@dataclass
class Qwen2Cfg:
    num_layers: int
    hidden: int
    heads: int
    kv_heads: int
    intermediate: int
    vocab: int
    tie_word_embeddings: bool = True
    eps: float = 1e-6
    final_eps: float = 1e-5
    theta: float = 1e6
    table_dtype: torch.dtype = torch.float16  # storage of the cos/sin table (pre_layer.py:30)

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads  # model.py:19


class Qwen2Oracle:
    def __init__(self, cfg: Qwen2Cfg, sd: dict, dtype: torch.dtype, max_batch: int,
                 max_length: int, kv_slots: int, quant: str = None):
        """quant="w8a8": every layer projection is int8 x int8 -> int32 with
        per-channel weight scales (quantize_weight_per_channel_absmax on the
        dtype-rounded weight, smooth_quant/layer.py:5-16) and dynamic
        per-token activation scales, dequantised in fp32 before the bias;
        lm_head stays in the model dtype (smooth_quant/qwen2.py:249-250).
        An int8 state dict (the SmoothQuant converter's output) supplies the
        int8 weights and scales itself, and a projection with a quant_scale
        quantises its input statically with that scale."""
        self.cfg, self.dtype, self.quant = cfg, dtype, quant
        r = lambda t: ops.rnd(t.detach().cpu(), dtype)  # noqa: E731
        self.embed = r(sd["model.embed_tokens.weight"])
        self.lm_head = self.embed if cfg.tie_word_embeddings else r(sd["lm_head.weight"])
        self.norm = r(sd["model.norm.weight"])
        self.layers = []
        int8 = sd["model.layers.0.self_attn.q_proj.weight"].dtype == torch.int8
        assert not int8 or quant == "w8a8", "an int8 checkpoint runs with quant='w8a8'"
        for i in range(cfg.num_layers):
            p = f"model.layers.{i}."
            if int8:
                # converter output (smooth_quant/layer.py:19-94): int8 weight,
                # weight_scale [out, 1] in its stored dtype, quant_scale = static
                # input scale where present; biases and norms stay float
                w = dict(bq=r(sd[p + "self_attn.q_proj.bias"]), bk=r(sd[p + "self_attn.k_proj.bias"]),
                         bv=r(sd[p + "self_attn.v_proj.bias"]),
                         ln1=r(sd[p + "input_layernorm.weight"]),
                         ln2=r(sd[p + "post_attention_layernorm.weight"]))
                for nm, mod in (("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"),
                                ("wv", "self_attn.v_proj"), ("wo", "self_attn.o_proj"),
                                ("wg", "mlp.gate_proj"), ("wu", "mlp.up_proj"),
                                ("wd", "mlp.down_proj")):
                    w[nm + "_i8"] = (sd[p + mod + ".weight"],
                                     sd[p + mod + ".weight_scale"].reshape(-1))
                    if sd.get(p + mod + ".quant_scale") is not None:
                        w[nm + "_as"] = sd[p + mod + ".quant_scale"]
                self.layers.append(w)
                continue
            self.layers.append(dict(
                wq=r(sd[p + "self_attn.q_proj.weight"]), bq=r(sd[p + "self_attn.q_proj.bias"]),
                wk=r(sd[p + "self_attn.k_proj.weight"]), bk=r(sd[p + "self_attn.k_proj.bias"]),
                wv=r(sd[p + "self_attn.v_proj.weight"]), bv=r(sd[p + "self_attn.v_proj.bias"]),
                wo=r(sd[p + "self_attn.o_proj.weight"]),
                wg=r(sd[p + "mlp.gate_proj.weight"]), wu=r(sd[p + "mlp.up_proj.weight"]),
                wd=r(sd[p + "mlp.down_proj.weight"]),
                ln1=r(sd[p + "input_layernorm.weight"]),
                ln2=r(sd[p + "post_attention_layernorm.weight"]),
            ))
        if quant == "w8a8" and not int8:
            for w in self.layers:
                for name in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
                    w[name + "_i8"] = ops.quantize_weight_per_channel_absmax(w[name].to(dtype))
        D, KVH = cfg.head_dim, cfg.kv_heads
        self.pool = torch.zeros((cfg.num_layers, kv_slots, 2 * KVH, D), dtype=ops.compute_dtype())
        self.cache = PageCache(max_batch, max_length, kv_slots)
        cos, sin = ops.rope_table(max_length, D, cfg.theta, cfg.table_dtype)
        self.cos, self.sin = cos.to(ops.compute_dtype()), sin.to(ops.compute_dtype())

    def _linear(self, x, w, names, bias=None):
        if self.quant != "w8a8":
            if len(names) == 1:
                wt = w[names[0]]
            else:  # the concatenated [gate; up] weight, built once
                key = "+".join(names)
                if key not in w:
                    w[key] = torch.cat([w[n] for n in names], 0)
                wt = w[key]
            return ops.linear(x, wt, bias)
        sa = w.get(names[0] + "_as")  # static input scale (o_proj, down_proj of a converted model)
        if sa is not None:
            xq, st = ops.quantize_static(x.to(self.dtype), sa)
        else:
            xq, st = ops.quantize_per_token_absmax(x.to(self.dtype))
        wq = torch.cat([w[n + "_i8"][0] for n in names], 0)
        so = torch.cat([w[n + "_i8"][1] for n in names], 0)
        y = ops.dequant_int32(ops.int8_gemm_i32(xq, wq), st, so).to(ops.compute_dtype())
        return y if bias is None else y + bias

    # ------------------------------------------------------------ one forward
    def forward(self, reqs, is_prefill: bool, ids):
        cfg, dt = self.cfg, self.dtype
        H, KVH, D = cfg.heads, cfg.kv_heads, cfg.head_dim
        _, pos, start, lens, shared, rids = no_padding_messages(reqs, is_prefill)
        if is_prefill:
            mem = self.cache.alloc_token_idxs(rids, shared, [l - s for l, s in zip(lens, shared)])
        else:
            mem = self.cache.alloc_token_idxs(rids, [l - 1 for l in lens], [1] * len(reqs))
        mem = torch.as_tensor(mem).long()
        r2t = torch.as_tensor(self.cache.req_to_tokens_)
        pos_t = torch.as_tensor(pos).long()
        cos, sin = self.cos[pos_t], self.sin[pos_t]
        T = len(ids)
        h = self.embed[torch.as_tensor(ids).long()]
        for li, w in enumerate(self.layers):
            x = ops.rnd(ops.rmsnorm(h, w["ln1"], cfg.eps), dt)
            q = ops.rnd(self._linear(x, w, ["wq"], w["bq"]), dt).view(T, H, D)
            k = ops.rnd(self._linear(x, w, ["wk"], w["bk"]), dt).view(T, KVH, D)
            v = ops.rnd(self._linear(x, w, ["wv"], w["bv"]), dt).view(T, KVH, D)
            q = ops.rnd(ops.rotary(q, cos, sin), dt)
            k = ops.rnd(ops.rotary(k, cos, sin), dt)
            self.pool[li, mem, :KVH] = k
            self.pool[li, mem, KVH:] = v
            kp, vp = self.pool[li, :, :KVH], self.pool[li, :, KVH:]
            if is_prefill:
                a = ops.prefill_attention(q, kp, vp, rids, start, lens, r2t,
                                          b_shared_seq_len=shared, p_dtype=dt)
            else:
                a = ops.decode_attention(q, r2t, rids, lens, kp, vp)
            a = ops.rnd(a, dt).view(T, H * D)
            o = ops.rnd(self._linear(a, w, ["wo"]), dt)
            h = ops.rnd(h + o, dt)
            x2 = ops.rnd(ops.rmsnorm(h, w["ln2"], cfg.eps), dt)
            gu = ops.rnd(self._linear(x2, w, ["wg", "wu"]), dt)
            act = ops.rnd(ops.silu_and_mul(gu, dt), dt)
            f = ops.rnd(self._linear(act, w, ["wd"]), dt)
            h = ops.rnd(h + f, dt)
        if is_prefill:  # last row of each request (post_layer.py:26-41)
            rows = [st + (l - s) - 1 for st, l, s in zip(start, lens, shared)]
        else:
            rows = list(start)
        hs = ops.rnd(ops.rmsnorm(h[torch.as_tensor(rows)], self.norm, cfg.final_eps), dt)
        logits = ops.linear(hs, self.lm_head)  # not rounded to dt: fp32 logits
        return ops.argmax_first(logits), logits

    # ------------------------------------------------------------ greedy loop
    def generate(self, prompts, n_new: int, return_logits: bool = False, feed=None, prefix=None):
        """Prefill all prompts as one NoPad batch, then n_new-1 decode steps
        (the loop of test/generate_token.py:61-63). Returns [B, n_new] tokens.

        feed [B, >= n_new-1] (optional): the tokens appended after each step
        instead of this oracle's own argmax (teacher forcing), so that every
        step is evaluated on the same context as the run that produced them;
        the returned tokens are still this oracle's argmax at each step.

        prefix (optional): a token list prefilled first as a request of its
        own; every prompt that extends it then starts from its slots as a
        shared prefix and prefills only its suffix (prompt-cache prefill,
        flash_attn_v2.py:699-762), which equals the full causal prefill of the
        prompt because a prefix token's K/V depend on the prefix alone."""
        pslots = None
        if prefix is not None:
            pre = Req(rid=self.cache.alloc_req(), input_tokens=list(prefix))
            self.forward([pre], True, list(prefix))
            pslots = self.cache.req_to_tokens_[pre.rid, :len(prefix)].copy()
        reqs = []
        for p in prompts:
            rid = self.cache.alloc_req()
            p = list(p)
            if pslots is not None and len(p) > len(prefix) and p[:len(prefix)] == list(prefix):
                self.cache.add_refs(rid, pslots)
                reqs.append(Req(rid=rid, input_tokens=p[len(prefix):], shared_tokens=list(prefix)))
            else:
                reqs.append(Req(rid=rid, input_tokens=p))
        ids = [t for r in reqs for t in r.input_tokens]
        toks, logits = self.forward(reqs, True, ids)
        out, all_logits = [toks], [logits]
        for i in range(n_new - 1):
            nxt = toks.tolist() if feed is None else [int(t) for t in feed[:, i]]
            for r, t in zip(reqs, nxt):
                r.output_tokens.append(t)
            toks, logits = self.forward(reqs, False, nxt)
            out.append(toks)
            all_logits.append(logits)
        res = torch.stack(out, 1)
        return (res, torch.stack(all_logits, 1)) if return_logits else res
