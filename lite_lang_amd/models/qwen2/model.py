"""Qwen2 model and runner on the lite_lang_amd kernels.

Counterpart of litelang/models/qwen2/model.py (Qwen2Model :23-97,
Qwen2ModelRunner :100-175) and of the layer modules it drives
(layer/pre_layer.py, layer/transformer_layer.py, layer/post_layer.py). The
runner API is the reference's; the layer body is the reference dataflow with
these fusions, each bit-identical to the unfused sequence:
  * residual add + RMSNorm in one kernel (transformer_layer.py:69-71,76 + :61);
  * q/k/v in one GEMM over the concatenated [q; k; v] rows;
  * RoPE of q and k + KV-pool scatter in one kernel reading cos/sin by
    position (transformer_layer.py:102-115,142-143);
  * the final residual add is applied only to the rows the post layer keeps
    (post_layer.py:26-41), fused with the final RMSNorm.
"""
from __future__ import annotations

import numpy as np
import torch

from lite_lang_amd import ops
from lite_lang_amd.models.cache import PageCache
from lite_lang_amd.models.radix_cache import RadixTree
from .decode_graph import DecodeGraph
from .weights import (DeviceWeights, Qwen2Config, check_smoothquant_config, is_int8_checkpoint,
                      load_state_dict, random_state_dict)


def rope_tables(max_length: int, head_dim: int, theta: float, device):
    """cos/sin [max_length, D/2]: built in fp32 on the host and rounded to fp16
    like Qwen2PreLayer._ComputePosition (pre_layer.py:21-30); kept as fp32
    values on the device so every model dtype sees the same table."""
    freqs = 1.0 / theta ** (torch.arange(0, head_dim, 2) / head_dim)
    ang = torch.arange(0, max_length)[:, None] * freqs[None, :]
    cos = torch.cos(ang).to(torch.float16).to(torch.float32)
    sin = torch.sin(ang).to(torch.float16).to(torch.float32)
    return cos.to(device).contiguous(), sin.to(device).contiguous()


def dense(x, w, bias=None):
    """Projection of the generic (prefill) path: ll_gemm, which runs the
    256 x 256 MFMA tile kernel above 64 rows and the weight-streaming kernel
    at or below (transformer_layer.py:80,82,95-109)."""
    return ops.gemm(x, w, bias)


class Qwen2Model:
    def __init__(self, layer_nums, max_length, config: Qwen2Config, tp_rank=0, world_size=1,
                 dtype=torch.bfloat16, device="cuda", quant=None):
        assert world_size == 1, "this build runs tp=1 (one GPU, no collectives)"
        assert layer_nums == config.layer_nums
        assert quant in (None, "w8a8"), f"unknown quantisation {quant!r}"
        self.cfg = config
        self.dtype = dtype
        self.quant = quant
        self.fuse_norm_qkv = True  # add + RMSNorm + next QKV in one decode launch
        self.device = torch.device(device)
        self.max_length = max_length
        self.cos, self.sin = rope_tables(max_length, config.head_dim, config.rope_theta,
                                         self.device)
        self.w: DeviceWeights | None = None
        self.last_logits = None  # logits of the latest forward (inspection only)

    def load_state_dict(self, sd):
        self.w = DeviceWeights(self.cfg, sd, self.dtype, self.device, quant=self.quant)

    def _proj(self, x, li, name, bias=None):
        """One layer projection in the generic path (bf16 GEMM or W8A8)."""
        if self.quant == "w8a8":
            return ops.linear_w8a8(x, self.w.packed[li][name + "_i8"], bias)
        return dense(x, self.w.layers[li][name], bias)

    def _gate_up_silu(self, x, li):
        """silu(x @ gate^T) * (x @ up^T) (transformer_layer.py:95-109). Above
        64 rows, when the weights have an interleaved copy, in one tile GEMM
        whose epilogue applies SiLU_and_Mul (bit-identical to the product
        followed by silu_and_mul); otherwise the [M, 2I] product, then
        silu_and_mul into a contiguous [M, I] buffer."""
        T = x.shape[0]
        if T > 64:
            if self.quant == "w8a8":
                qw = self.w.packed[li]["wgu_i8"]
                if qw.q_il is not None and x.dtype in (torch.bfloat16, torch.float16):
                    xq, st = ops.quant_input(x, qw)
                    return ops.gemm_i8_gate_up_silu_tiled(xq, st, qw.q_il, qw.scale,
                                                          out_dtype=x.dtype)
            else:
                w_il = self.w.layers[li].get("wgu_il")
                if w_il is not None:
                    return ops.gate_up_silu_tiled(x, w_il)
        gu = self._proj(x, li, "wgu")
        return ops.silu_and_mul(gu, out=torch.empty((T, gu.shape[1] // 2), dtype=gu.dtype,
                                                    device=gu.device))

    # ------------------------------------------------------------ layer stack
    def _layers(self, h, T, slots, positions, pool, attention):
        """The L transformer layers (transformer_layer.py:46-77) over hidden
        rows h [T, hidden] (updated in place with the attention residual and
        all but the last FFN residual). Returns the last FFN output."""
        cfg, w = self.cfg, self.w
        H, KVH, D = cfg.num_heads, cfg.num_key_value_heads, cfg.head_dim
        attn = torch.empty((T, H, D), dtype=self.dtype, device=self.device)
        f = None
        for li, lw in enumerate(w.layers):
            x = ops.rmsnorm(h, lw["ln1"], cfg.rms_norm_eps, residual=f)
            qkv = self._proj(x, li, "wqkv", lw["bqkv"])
            ops.rope_kv_scatter(qkv, H, KVH, D, positions, self.cos, self.sin, slots, pool[li])
            q = qkv[:, : H * D].view(T, H, D)
            attention(li, q, attn)
            o = self._proj(attn.view(T, H * D), li, "wo")
            x2 = ops.rmsnorm(h, lw["ln2"], cfg.rms_norm_eps, residual=o)
            act = self._gate_up_silu(x2, li)
            f = self._proj(act, li, "wdown")
        return f

    def _logits(self, x):
        """lm_head (post_layer.py:20-22). With 16-bit weights and at most 64
        rows (decode; the last rows of a prefill), the packed weight stream
        writes the logits in fp32, unrounded, and the argmax reads those (the
        reference argmaxes its fp16 logits, post_layer.py:75-77; bf16 logits
        would tie where fp16 ones do not). Otherwise the model dtype."""
        w = self.w
        if w.lm_head_p is not None and x.shape[0] <= 64:
            return ops.gemm_packed(x, w.lm_head_p, out_dtype=torch.float32)
        return ops.gemm(x, w.lm_head)

    def _logits_argmax(self, x, out, status=None):
        """lm_head + greedy pick of the decode step: the fused call (the
        argmax's first pass in the lm_head's epilogue) where the packed lm_head
        applies, else _logits and ll_argmax. Sets last_logits; returns the
        tokens (in `out` when given)."""
        w = self.w
        if w.lm_head_p is not None and x.shape[0] <= 64:
            logits, toks = ops.gemm_packed_argmax(x, w.lm_head_p, out=out, status=status)
        else:
            logits = self._logits(x)
            toks = ops.argmax(logits, out=out, status=status)
        self.last_logits = logits
        return toks

    def _post(self, hs, fs, out=None):
        """Final residual add + RMSNorm (eps 1e-5), lm_head, greedy argmax
        (post_layer.py:14-24,43-45,75-77)."""
        y = ops.rmsnorm(hs, self.w.norm, self.cfg.final_norm_eps, residual=fs)
        logits = self._logits(y)
        self.last_logits = logits
        return ops.argmax(logits, out=out)

    # ------------------------------------------------------------ decode
    def _proj_shapes(self):
        cfg = self.cfg
        H, KVH, D, hd, I = (cfg.num_heads, cfg.num_key_value_heads, cfg.head_dim,
                            cfg.hidden_size, cfg.intermediate_size)
        return [((H + 2 * KVH) * D, hd), (hd, H * D), (2 * I, hd), (hd, I)]

    def splitk_part_numel(self, batch):
        """fp32 elements of the partial-sum buffer the fused decode path needs
        (W8A8: one dequantised split)."""
        if self.quant == "w8a8":
            return max(batch * n for n, _ in self._proj_shapes())
        need = max(ops.gemm_splitk_count(batch, n, k) * batch * n for n, k in self._proj_shapes())
        qs = self.norm_qkv_splits(batch)
        return max(need, qs * batch * self._proj_shapes()[0][0])

    def norm_qkv_splits(self, batch):
        """QKV split count of the add + RMSNorm + QKV launch of the fused
        decode layer (ops.add_rmsnorm_qkv_splitk), 0 where it does not apply:
        it needs the packed QKV weight of every layer and a shape the kernel
        covers; fuse_norm_qkv = False turns it off."""
        if not self.fuse_norm_qkv or self.quant == "w8a8" or not self.fused_decode_ok(batch):
            return 0
        if self.w is None or any(pk.get("wqkv") is None for pk in self.w.packed):
            return 0
        n, k = self._proj_shapes()[0]
        return ops.add_rmsnorm_qkv_splits(batch, k, n)

    def w8a8_part_bytes(self, batch):
        """int32 partial bytes of the W8A8 projections at this batch size."""
        return max(ops.gemm_i8_splitk_count(batch, n, k) * batch * n * 4
                   for n, k in self._proj_shapes())

    def _fused_rope_ok(self):
        cfg = self.cfg
        return cfg.head_dim in (64, 128) and cfg.num_heads // cfg.num_key_value_heads <= 16

    def _rope_attention(self, part, splits, bias, q, attn, positions, slots, pool_layer, r2t,
                        rids, seq_len, max_len):
        """RoPE + new-token K/V write + decode attention from the QKV split-K
        partials: one fused launch (plus the split merge) where the kernel
        covers the shape, else the scatter kernel followed by attention."""
        cfg = self.cfg
        H, KVH, D = cfg.num_heads, cfg.num_key_value_heads, cfg.head_dim
        if self._fused_rope_ok():
            ops.decode_attention_rope_splitk(part, splits, bias, positions, self.cos, self.sin,
                                             slots, r2t, rids, seq_len, max_len,
                                             pool_layer[:, :KVH], pool_layer[:, KVH:], attn)
            return
        B = attn.shape[0]
        ops.rope_kv_scatter_splitk(part, splits, bias, q, H, KVH, D, positions, self.cos, self.sin,
                                   slots, pool_layer)
        ops.decode_attention(q.view(B, H, D), r2t, rids, seq_len, max_len, pool_layer[:, :KVH],
                             pool_layer[:, KVH:], attn)

    def fused_decode_ok(self, batch):
        return self.dtype in (torch.bfloat16, torch.float16) and 0 < batch <= 64

    def decode_tokens(self, ids, positions, seq_len, rids, slots, kv_cache: PageCache, max_len,
                      out=None, slot_write=None):
        """One decode forward from device-resident metadata only (no host
        reads, so it can be captured in a HIP graph). ids/positions/seq_len
        [B] int32 or int64, rids/slots [B] int32; max_len bounds seq_len.
        Writes the next tokens [B] int64 into `out` (may alias ids).

        bf16/fp16 with B <= 64 runs the fused split-K layer: the projections
        leave fp32 partials that the next kernel finishes (RoPE + KV scatter,
        residual + RMSNorm) and the gate/up projection applies SiLU_and_Mul in
        its own epilogue, 8 launches per layer; other cases run the generic
        layer.

        slot_write: the step's slot-table update (int32 [3, >= B]: slots,
        request rows, columns), done first: by the step's first launch where
        that is the embedding + RMSNorm + epoch launch, else by assign_slots."""
        cfg = self.cfg
        H, KVH, D = cfg.num_heads, cfg.num_key_value_heads, cfg.head_dim
        B = ids.shape[0]
        pool, r2t = kv_cache.kv_cache_, kv_cache.req_to_tokens_
        fuse_qkv = self.fused_decode_ok(B) and self.quant != "w8a8" and self.norm_qkv_splits(B) > 0
        if slot_write is not None and not fuse_qkv:
            ops.assign_slots(r2t, slot_write, B)
        if not self.fused_decode_ok(B):
            h = ops.embedding(self.w.embed, ids)

            def attention(li, q, attn):
                ops.decode_attention(q, r2t, rids, seq_len, max_len, pool[li, :, :KVH],
                                     pool[li, :, KVH:], attn)

            f = self._layers(h, B, slots, positions, pool, attention)
            return self._post(h, f, out=out)

        w = self.w
        dev, dt = self.device, self.dtype
        part = ops.workspace(dev, "splitk_part", self.splitk_part_numel(B) * 4).view(torch.float32)
        q = torch.empty((B, H * D), dtype=dt, device=dev)
        attn = torch.empty((B, H, D), dtype=dt, device=dev)
        act = torch.empty((B, cfg.intermediate_size), dtype=dt, device=dev)
        nl = len(w.layers)
        if self.quant == "w8a8":
            h = ops.embedding(w.embed, ids)
            return self._decode_w8a8(h, B, part, q, attn, act, positions, seq_len, rids, slots,
                                     pool, r2t, max_len, out)
        # layers after the first take their QKV partials from the launch that
        # finishes the previous layer (residual + RMSNorm + QKV projection);
        # those launches tell this step's flags by the epoch, which the
        # step's first launch advances
        epoch = ops.decode_epoch(dev) if fuse_qkv else None
        h, x = ops.embedding_rmsnorm(w.embed, ids, w.layers[0]["ln1"], cfg.rms_norm_eps,
                                     epoch=epoch,
                                     slot_write=(r2t, slot_write) if fuse_qkv and slot_write
                                     is not None else None)

        def proj(xin, lw, pk, name):
            if pk.get(name) is not None:
                return ops.gemm_splitk_packed(xin, pk[name], part)
            return ops.gemm_splitk(xin, lw[name], part)

        qkv_s = None
        for li, (lw, pk) in enumerate(zip(w.layers, w.packed)):
            s = qkv_s if qkv_s is not None else proj(x, lw, pk, "wqkv")
            self._rope_attention(part, s, lw["bqkv"], q, attn, positions, slots, pool[li], r2t,
                                 rids, seq_len, max_len)
            s = proj(attn.view(B, H * D), lw, pk, "wo")
            x2 = ops.add_rmsnorm_splitk(h, part, s, lw["ln2"], cfg.rms_norm_eps)
            if pk.get("wgu_silu") is not None:
                ops.gate_up_silu(x2, pk["wgu_silu"], out=act)
            else:
                s = proj(x2, lw, pk, "wgu")
                ops.silu_and_mul_splitk(part, s, act)
            s = proj(act, lw, pk, "wdown")
            if li + 1 < nl and fuse_qkv:
                x, qkv_s = ops.add_rmsnorm_qkv_splitk(h, part, s, w.layers[li + 1]["ln1"],
                                                      cfg.rms_norm_eps, w.packed[li + 1]["wqkv"],
                                                      part, epoch, li)
            elif li + 1 < nl:
                x = ops.add_rmsnorm_splitk(h, part, s, w.layers[li + 1]["ln1"], cfg.rms_norm_eps)
            else:
                x = ops.add_rmsnorm_splitk(h, part, s, w.norm, cfg.final_norm_eps)
        # a fused launch that gave up a bounded wait (a flag wait of the norm +
        # QKV launch, the attention's split merge) turns every token into -1
        # (the host raises on it, runner_batch.check_step_tokens)
        return self._logits_argmax(x, out, ops.decode_sync_error(dev))

    def _decode_w8a8(self, h, B, part, q, attn, act, positions, seq_len, rids, slots, pool, r2t,
                     max_len, out):
        """The fused decode layer with int8 projections (9 launches per layer):
        each int8 GEMM leaves int32 partials that the next kernel dequantises
        inline (fused RoPE attention, add+RMSNorm), the gate/up GEMM applies
        dequantisation and SiLU_and_Mul in its own epilogue, and the
        attention's split merge and add+RMSNorm also emit the int8 input of
        the following projection (per token, or with the static scale of a
        converted checkpoint's o_proj). The SiLU product is quantised by its
        own vectorised kernel: a row-per-workgroup fusion measured slower (40
        CUs cannot pull the row's int32 partials as fast as the elementwise
        kernel spread over all of them)."""
        cfg, w = self.cfg, self.w
        H, KVH, D = cfg.num_heads, cfg.num_key_value_heads, cfg.head_dim
        nl = len(w.layers)

        def fused_quant(pk, name):
            return pk[name + "_i8"].input_scale is None

        x = ops.rmsnorm(h, w.layers[0]["ln1"], cfg.rms_norm_eps)
        xq, xs = ops.quant_input(x, w.packed[0]["wqkv_i8"])
        for li, (lw, pk) in enumerate(zip(w.layers, w.packed)):
            p = ops.gemm_w8a8_i32(xq, xs, pk["wqkv_i8"])
            if self._fused_rope_ok():
                _, aq, as_ = ops.decode_attention_rope_splitk_i32(
                    p, lw["bqkv"], positions, self.cos, self.sin, slots, r2t, rids, seq_len,
                    max_len, pool[li, :, :KVH], pool[li, :, KVH:], attn, quant=True,
                    input_scale=pk["wo_i8"].input_scale)
            else:
                n = p.s_ch.numel()
                ops.dequant_splitk(p.part, p.splits, p.s_tok, p.s_ch, part[: B * n].view(B, n),
                                   B, n)
                self._rope_attention(part, 1, lw["bqkv"], q, attn, positions, slots, pool[li],
                                     r2t, rids, seq_len, max_len)
                aq, as_ = ops.quant_input(attn.view(B, H * D), pk["wo_i8"])
            p = ops.gemm_w8a8_i32(aq, as_, pk["wo_i8"])
            if fused_quant(pk, "wgu"):
                _, x2q, x2s = ops.add_rmsnorm_splitk_i32(h, p, lw["ln2"], cfg.rms_norm_eps,
                                                         quant=True)
            else:
                x2 = ops.add_rmsnorm_splitk_i32(h, p, lw["ln2"], cfg.rms_norm_eps)
                x2q, x2s = ops.quant_input(x2, pk["wgu_i8"])
            if pk["wgu_i8"].packed_gu is not None:
                ops.gemm_i8_gate_up_silu(x2q, x2s, pk["wgu_i8"].packed_gu, act)
            else:
                ops.silu_and_mul_splitk_i32(ops.gemm_w8a8_i32(x2q, x2s, pk["wgu_i8"]), act)
            dq, ds = ops.quant_input(act, pk["wdown_i8"])
            p = ops.gemm_w8a8_i32(dq, ds, pk["wdown_i8"])
            if li + 1 < nl:
                nxt = w.packed[li + 1]
                if fused_quant(nxt, "wqkv"):
                    x, xq, xs = ops.add_rmsnorm_splitk_i32(
                        h, p, w.layers[li + 1]["ln1"], cfg.rms_norm_eps, quant=True)
                else:
                    x = ops.add_rmsnorm_splitk_i32(h, p, w.layers[li + 1]["ln1"],
                                                   cfg.rms_norm_eps)
                    xq, xs = ops.quant_input(x, nxt["wqkv_i8"])
            else:
                x = ops.add_rmsnorm_splitk_i32(h, p, w.norm, cfg.final_norm_eps)
        return self._logits_argmax(x, out)

    # ------------------------------------------------------------ forward
    def forward(self, model_inputs, kv_cache: PageCache, mem_idxs: torch.Tensor):
        """One forward of the NoPad batch; returns next tokens [B, 1] int64."""
        if not model_inputs.is_prefill:
            lens = model_inputs.host[3]
            return self.decode_tokens(model_inputs.output_token_ids, model_inputs.position_ids,
                                      model_inputs.b_seq_len, model_inputs.b_rids, mem_idxs,
                                      kv_cache, max(lens)).view(-1, 1)
        cfg = self.cfg
        KVH = cfg.num_key_value_heads
        _, _, start_h, lens_h, shared_h, _ = model_inputs.host
        ids = model_inputs.input_tokens
        T = ids.shape[0]
        pool, r2t = kv_cache.kv_cache_, kv_cache.req_to_tokens_
        max_len = max(lens_h)
        shared = model_inputs.b_shared_seq_len if model_inputs.radix_cache is not None else None
        h = ops.embedding(self.w.embed, ids)

        def attention(li, q, attn):
            ops.prefill_attention(q, pool[li, :, :KVH], pool[li, :, KVH:], attn,
                                  model_inputs.b_rids, model_inputs.b_start_idx,
                                  model_inputs.b_seq_len, max_len, r2t, b_shared_seq_len=shared)

        f = self._layers(h, T, mem_idxs, model_inputs.position_ids, pool, attention)
        # last row of each request (post_layer.py:26-41)
        rows = [s + (l - sh) - 1 for s, l, sh in zip(start_h, lens_h, shared_h)]
        rows_d = torch.from_numpy(np.asarray(rows, dtype=np.int64)).pin_memory().to(
            self.device, non_blocking=True)
        return self._post(ops.embedding(h, rows_d), ops.embedding(f, rows_d)).view(-1, 1)


class Qwen2ModelRunner:
    """Runner with the reference constructor and methods (model.py:100-175).

    Extra keyword arguments (all optional): dtype (default bfloat16),
    kv_max_size (token slots; default sized from free memory x mem_usage as
    the reference), state_dict (weights as a HF-style dict), seed (random
    init when neither model_path nor state_dict is given), device,
    use_cuda_graph (default True: decode steps replay a HIP graph captured
    once per batch size; the returned token tensor is then valid until the
    next forward).
    """

    def __init__(self, layer_nums, max_batch_size, config: Qwen2Config, **runner_kwargs):
        self.tp_rank_ = runner_kwargs.get("tp_rank", 0)
        self.world_size_ = runner_kwargs.get("world_size", 1)
        assert self.world_size_ == 1, "this build runs tp=1 (one GPU, no collectives)"
        self.dtype_ = runner_kwargs.get("dtype", torch.bfloat16)
        self.device_ = torch.device(runner_kwargs.get("device", "cuda"))
        self.model_ins_ = Qwen2Model(layer_nums, runner_kwargs["max_length"], config,
                                     self.tp_rank_, self.world_size_, self.dtype_, self.device_,
                                     quant=runner_kwargs.get("quant"))
        self.model_path_ = runner_kwargs.get("model_path")
        self.state_dict_ = runner_kwargs.get("state_dict")
        self.seed_ = runner_kwargs.get("seed", 0)
        self.kv_max_size_arg_ = runner_kwargs.get("kv_max_size")
        self.max_batch_size_ = max_batch_size
        self.max_length_ = runner_kwargs["max_length"]
        self.mem_usage_ = runner_kwargs.get("mem_usage", 0.5)
        self.use_radix_cache_ = runner_kwargs.get("use_radix_cache", False)
        self.radix_cache = None
        self.kv_cache = None
        self.layer_nums_ = layer_nums
        self.config_ = config
        self.use_cuda_graph_ = runner_kwargs.get("use_cuda_graph", True)
        self._graphs = {}

    def init_model(self):
        """Load the weights, allocate the KV pool; returns its size in token
        slots. A second call returns the same size and changes nothing (the
        weights a state dict supplied are not kept, so they could not be
        loaded again)."""
        if self.kv_cache is not None:
            return self.kv_cache.kv_max_size_
        if self.state_dict_ is not None:
            sd = self.state_dict_
        elif self.model_path_:
            sd = load_state_dict(self.model_path_)
            if is_int8_checkpoint(sd):
                # the SmoothQuant converter's output runs on the W8A8 runtime
                check_smoothquant_config(self.model_path_)
                if self.model_ins_.quant is None:
                    self.model_ins_.quant = "w8a8"
        else:
            sd = random_state_dict(self.config_, seed=self.seed_, device=self.device_,
                                   dtype=self.dtype_)
        self.model_ins_.load_state_dict(sd)
        self.state_dict_ = None
        self.kv_cache = PageCache(self.max_batch_size_, self.max_length_, self.mem_usage_,
                                  self.layer_nums_, self.config_.head_dim,
                                  self.config_.num_key_value_heads, torch_dtype=self.dtype_,
                                  tp_rank=self.tp_rank_, tp_world_size=self.world_size_,
                                  kv_max_size=self.kv_max_size_arg_, device=self.device_)
        self.radix_cache = RadixTree() if self.use_radix_cache_ else None
        self._check_merge_premise()
        return self.kv_cache.kv_max_size_

    def _check_merge_premise(self):
        """Decode attention merges its splits inside the split stage only
        where all workgroups of a sequence share an XCD (the dispatcher's
        round-robin gives that). Checked once on this machine at the decode
        shape; when it does not hold, every decode attention call of the
        process merges in a separate kernel instead."""
        cfg = self.config_
        self.same_launch_merge = ops.decode_attention_xcd_premise(
            self.device_, min(self.max_batch_size_, 64), cfg.num_heads,
            cfg.num_key_value_heads, cfg.head_dim, self.max_length_)
        if not self.same_launch_merge:
            ops.set_same_launch_merge(False)

    def reset_decode_fault(self):
        """Clear the error word a fused decode launch sets when it gives up a
        bounded wait (on the decode graphs' stream and on the current stream);
        until then every decode step returns token ids of -1. The decode
        attention's workspace is zeroed too: a split merge that gave up may
        have left partial words that the next merge would take as written."""
        from .decode_graph import _capture_stream
        with torch.cuda.stream(_capture_stream(self.device_)):
            ops.decode_sync_status(self.device_, reset=True)
            ops.clear_workspace(self.device_, "decode_attention")
        ops.decode_sync_status(self.device_, reset=True)
        ops.clear_workspace(self.device_, "decode_attention")

    def _alloc_for_forward(self, model_inputs):
        """Slot allocation done by layer 0 in the reference (transformer_layer.py:53-60)."""
        _, _, _, lens, shared, rids = model_inputs.host
        if model_inputs.is_prefill:
            match = [len(r.match_token_idxs) if r.match_token_idxs is not None else 0
                     for r in model_inputs.request_mapping.values()]
            return self.kv_cache.alloc_token_idxs(rids, match, [l - m for l, m in zip(lens, match)])
        return self.kv_cache.alloc_token_idxs(rids, [l - 1 for l in lens], [1] * len(lens))

    def forward(self, model_inputs):
        if self.radix_cache is not None:
            self._compute_if_need_free_radix_tree(model_inputs)
        if not model_inputs.is_prefill and self.use_cuda_graph_:
            return self._graph_decode(model_inputs)
        mem_idxs = self._alloc_for_forward(model_inputs)
        return self.model_ins_.forward(model_inputs, self.kv_cache, mem_idxs)

    def _graph_decode(self, model_inputs):
        _, pos, _, lens, _, rids = model_inputs.host
        B = len(lens)
        g = self._graphs.get(B)
        if g is None:
            g = DecodeGraph(self.model_ins_, self.kv_cache, B, self.max_length_,
                            reserve_upto=self.max_batch_size_)
            self._graphs[B] = g
        slots, rows, cols = self.kv_cache.plan_token_idxs(rids, [l - 1 for l in lens], [1] * B)
        out = g.run(model_inputs.output_token_ids, slots, rows, cols, pos, lens)
        return out.view(-1, 1)

    def _compute_if_need_free_radix_tree(self, model_inputs):
        """Evict LRU radix leaves when the next forward needs more slots than
        are free (model.py:128-144)."""
        ids, _, _, lens, _, _ = model_inputs.host
        need_now = len(ids) if model_inputs.is_prefill else len(lens)
        need = self.kv_cache.if_need_more_tokens(need_now)
        token_idxs = self.radix_cache.evict_node(need)
        if token_idxs is not None:
            self.kv_cache.free_token_idxs(token_idxs)

    def _add_new_req(self, length):
        if self.kv_cache.can_allocated(length):
            return self.kv_cache.alloc_req()
        return None

    def free_reqs(self, reqs):
        if self.radix_cache is not None:
            return
        self.kv_cache.dealloc_reqs(reqs)
