"""HIP-graph replay of the decode step.

The reference rebuilds six metadata tensors on the host, reads 2*B scalars
back and launches every kernel from Python on each decode step
(runner_batch.py:227-243, transformer_layer.py:154); its README names the
resulting timeline gaps as the bottleneck (README.md:108-116). Here one
decode forward for a fixed batch size is captured once into a HIP graph:

  * per-step metadata (new slot ids, request rows, slot-table columns,
    positions, lengths) lives in one static int32 device buffer [5, B] that
    the host refreshes with a single pinned upload before each replay;
  * the slot-table write is done by the graph's first launch (the embedding
    + RMSNorm + epoch launch of the fused layer; ll_assign_slots of its own
    otherwise);
  * the argmax writes the next tokens straight into the static token buffer
    the embedding of the next replay reads, so consecutive steps chain on the
    device without a host round trip;
  * decode attention is captured with the runner's max_length as the length
    bound: its split count and workspace are fixed, and every sequence
    divides its own current length among the splits (ll_decode_attention).
Every decode graph of a device is captured on one stream of this module's
(_capture_stream), and the library workspaces that stream uses are reserved
on it before capture, so nothing is allocated by the library inside the
graph; activations come from the graph's private pool. The workspaces of
that stream are never freed (a larger capture retires a buffer instead), so
graphs captured earlier keep valid addresses.
"""
from __future__ import annotations

import numpy as np
import torch

from lite_lang_amd import _lib, ops


def reserve_decode_workspaces(cfg, batch, max_len, device):
    L = _lib.load()
    D, H, KVH = cfg.head_dim, cfg.num_heads, cfg.num_key_value_heads
    ops.reserve_workspace(device, "decode_attention",
                          L.ll_decode_attention_workspace_size(batch, H, KVH, D, max_len))
    shapes = [((H + 2 * KVH) * D, cfg.hidden_size), (cfg.hidden_size, H * D),
              (2 * cfg.intermediate_size, cfg.hidden_size),
              (cfg.hidden_size, cfg.intermediate_size), (cfg.vocab_size, cfg.hidden_size)]
    ops.reserve_workspace(device, "gemm",
                          max(L.ll_gemm_workspace_size(batch, n, k) for n, k in shapes))
    ops.reserve_workspace(device, "argmax", L.ll_argmax_workspace_size(batch, cfg.vocab_size))
    ops.reserve_workspace(device, "lm_argmax", L.ll_gemm_packed_f32_argmax_workspace_size(
        batch, cfg.vocab_size, cfg.hidden_size))


def reserve_model_workspaces(model, batch, max_len):
    reserve_decode_workspaces(model.cfg, batch, max_len, model.device)
    if model.fused_decode_ok(batch):
        ops.reserve_workspace(model.device, "splitk_part", model.splitk_part_numel(batch) * 4)
        ops.decode_sync(model.device)  # the error word of the fused launches' bounded waits
        if model.quant == "w8a8":
            ops.reserve_workspace(model.device, "w8a8_part", model.w8a8_part_bytes(batch))
        if model.norm_qkv_splits(batch) > 0:
            ops.reserve_workspace(model.device, "decode_epoch", 4)


_CAPTURE_STREAMS: dict[int, torch.cuda.Stream] = {}


def _capture_stream(device) -> torch.cuda.Stream:
    """The stream every decode graph of `device` is captured on (default priority)."""
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    s = _CAPTURE_STREAMS.get(idx)
    if s is None:
        s = torch.cuda.Stream(device=idx)
        _CAPTURE_STREAMS[idx] = s
    return s


class DecodeGraph:
    META_ROWS = 5  # slots, rids, cols, positions, seq_len

    def __init__(self, model, kv_cache, batch_size: int, max_len: int, reserve_upto: int = 0):
        """reserve_upto: also size the workspaces for batches up to this size
        (the runner's max batch), so later captures need no larger buffers."""
        self.model, self.kv_cache = model, kv_cache
        self.B = batch_size
        self.max_len = max_len
        dev = model.device
        self.meta = torch.zeros((self.META_ROWS, batch_size), dtype=torch.int32, device=dev)
        self.ids = torch.zeros((batch_size,), dtype=torch.int64, device=dev)
        self._host = [torch.zeros((self.META_ROWS, batch_size), dtype=torch.int32,
                                  pin_memory=True) for _ in range(2)]
        self._host_ev = [None, None]
        self._k = 0
        stream = _capture_stream(dev)
        with torch.cuda.stream(stream):
            for b in sorted({batch_size, min(reserve_upto, 64), reserve_upto} - {0}):
                reserve_model_workspaces(model, b, max_len)
        # the slot table must never be written by the capture itself
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            model.decode_tokens(self.ids, self.meta[3], self.meta[4], self.meta[1], self.meta[0],
                                kv_cache, max_len, out=self.ids, slot_write=self.meta[0:3])
        self.logits = model.last_logits  # the graph's own logits buffer
        torch.cuda.synchronize(dev)

    def run(self, in_ids: torch.Tensor, slots, rids, cols, positions, seq_len) -> torch.Tensor:
        """Upload this step's metadata, replay, return the token buffer [B]
        (valid until the next replay)."""
        i = self._k & 1
        self._k += 1
        if self._host_ev[i] is not None:
            self._host_ev[i].synchronize()
        hm = self._host[i].numpy()
        hm[0], hm[1], hm[2], hm[3], hm[4] = slots, rids, cols, positions, seq_len
        self.meta.copy_(self._host[i], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._host_ev[i] = ev
        if in_ids.data_ptr() != self.ids.data_ptr():
            self.ids.copy_(in_ids.view(-1))
        self.graph.replay()
        self.model.last_logits = self.logits
        return self.ids
