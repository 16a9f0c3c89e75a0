"""NoPad batch metadata and request bookkeeping.

Counterpart of litelang/models/runner_batch.py (get_no_padding_messages
:8-35, RunnerReq :38-85, RunnerBatch :88-265) with the same public API. The
metadata is built on the host from the request lists and uploaded in one
pinned copy (the reference makes six separate torch.tensor(...).cuda() calls
and 2*B .item() reads per step).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict

import numpy as np
import torch

from .cache import PageCache
from .radix_cache import RadixTree


def get_no_padding_messages_host(input_reqs, is_prefill=True):
    """Host lists (input_ids, position_ids, start_idx, seq_len, shared_len, rids)."""
    position_ids, input_ids, req_lengths, start_idx, shared_seq_len, rids = [], [], [], [], [], []
    for idx, req in enumerate(input_reqs):
        rids.append(req.rid)
        if is_prefill:
            ns = len(req.shared_tokens)
            shared_seq_len.append(ns)
            position_ids.extend(range(ns, ns + len(req.input_tokens)))
            start_idx.append(len(input_ids))
            input_ids.extend(req.input_tokens)
        else:
            position_ids.append(req.length - 1)
            start_idx.append(idx)
            shared_seq_len.append(len(req.shared_tokens))
        req_lengths.append(req.length)
    return input_ids, position_ids, start_idx, req_lengths, shared_seq_len, rids


def _upload(lists, device):
    """One pinned host buffer -> device; returns int64 device tensors, one per list."""
    sizes = [len(x) for x in lists]
    flat = np.zeros(max(1, sum(sizes)), dtype=np.int64)
    o = 0
    for x, n in zip(lists, sizes):
        flat[o:o + n] = x
        o += n
    dev = torch.from_numpy(flat).pin_memory().to(device, non_blocking=True)
    out, o = [], 0
    for n in sizes:
        out.append(dev[o:o + n])
        o += n
    return out


def get_no_padding_messages(input_reqs, is_prefill=True, device="cuda"):
    """Device tensors (input_ids, position_ids, b_start_idx, b_seq_len,
    b_shared_seq_len, b_rids) as in runner_batch.py:8-35 (b_rids int32)."""
    ids, pos, st, lens, shared, rids = get_no_padding_messages_host(input_reqs, is_prefill)
    t_ids, t_pos, t_st, t_len, t_sh, t_rid = _upload([ids, pos, st, lens, shared, rids], device)
    return t_ids, t_pos, t_st, t_len, t_sh, t_rid.to(torch.int32)


@dataclass
class RunnerReq:
    id: int
    rid: int
    input_length: int
    output_length: int = 0
    shared_tokens: list = None
    match_token_idxs: object = None
    input_tokens: list = None
    output_tokens: list = None
    temperature: float = 0.0
    top_p: float = 0.0
    top_k: float = 0.0
    do_sample: bool = False

    @staticmethod
    def create_runner_req(id, input_tokens, shared_tokens, match_token_idxs, temperature, top_p,
                          top_k, do_sample) -> "RunnerReq":
        return RunnerReq(id=id, rid=None, input_length=len(input_tokens),
                         shared_tokens=shared_tokens, match_token_idxs=match_token_idxs,
                         input_tokens=input_tokens, temperature=temperature, top_p=top_p,
                         top_k=top_k, do_sample=do_sample)

    @property
    def length(self):
        return len(self.shared_tokens) + self.input_length + self.output_length

    def update_forward_message(self, token_id):
        self.output_length += 1
        if self.output_tokens is None:
            self.output_tokens = []
        self.output_tokens.append(int(token_id))


@dataclass
class RunnerBatch:
    id: object
    request_mapping: Dict[int, RunnerReq]
    input_tokens: torch.Tensor
    position_ids: torch.Tensor
    b_start_idx: torch.Tensor
    b_seq_len: torch.Tensor
    b_shared_seq_len: torch.Tensor
    b_rids: torch.Tensor
    output_token_ids: torch.Tensor
    is_prefill: bool
    radix_cache: RadixTree
    kv_cache: PageCache
    host: tuple = None  # host lists of the current metadata

    def _refresh(self, is_prefill):
        device = self.kv_cache.device
        h = get_no_padding_messages_host(self.request_mapping.values(), is_prefill)
        t_ids, t_pos, t_st, t_len, t_sh, t_rid = _upload(list(h), device)
        self.input_tokens, self.position_ids, self.b_start_idx = t_ids, t_pos, t_st
        self.b_seq_len, self.b_shared_seq_len, self.b_rids = t_len, t_sh, t_rid.to(torch.int32)
        self.host = h

    @classmethod
    def create_batch(cls, req_messages, batch_id, is_prefill: bool = True, model_runner=None):
        """Admit requests (runner_batch.py:103-167): radix prefix match on all
        but the last prompt token, request-row allocation, shared-slot refs."""
        request_mapping = {}
        for message in req_messages:
            request_id = message["id"]
            input_tokens = list(message["input_tokens"])
            shared_tokens = []
            match_token_idxs, has_match_len = None, 0
            if model_runner.radix_cache is not None:
                match_token_idxs, has_match_len = model_runner.radix_cache.match_prefix(
                    torch.tensor(input_tokens[:-1], dtype=torch.int64))
                if has_match_len > 0:
                    shared_tokens = input_tokens[:has_match_len]
                    input_tokens = input_tokens[has_match_len:]
            new_req = RunnerReq.create_runner_req(
                id=request_id, input_tokens=input_tokens, shared_tokens=shared_tokens,
                match_token_idxs=match_token_idxs, temperature=message.get("temperature", 0.0),
                top_p=message.get("top_p", 0.0), top_k=message.get("top_k", 0.0),
                do_sample=message.get("do_sample", False))
            new_req.rid = model_runner._add_new_req(new_req.input_length)
            if model_runner.radix_cache is not None and new_req.match_token_idxs is not None:
                model_runner.kv_cache.add_refs(new_req.rid, new_req.match_token_idxs)
            request_mapping[request_id] = new_req
        batch = cls(id=batch_id, request_mapping=request_mapping, input_tokens=None,
                    position_ids=None, b_start_idx=None, b_seq_len=None, b_shared_seq_len=None,
                    b_rids=None, output_token_ids=None, is_prefill=is_prefill,
                    radix_cache=model_runner.radix_cache, kv_cache=model_runner.kv_cache)
        batch._refresh(is_prefill)
        return batch

    def get_post_sample_para(self):
        reqs = list(self.request_mapping.values())
        dev = self.kv_cache.device
        return (torch.tensor([r.temperature for r in reqs], device=dev),
                torch.tensor([r.top_p for r in reqs], device=dev),
                torch.tensor([r.top_k for r in reqs], device=dev),
                torch.tensor([r.do_sample for r in reqs], device=dev))

    def _free_req_cache(self, req_id):
        """Insert the finished request into the radix tree and release the
        duplicate slots and the request row (runner_batch.py:184-204)."""
        req = self.request_mapping[req_id]
        key = torch.tensor(req.shared_tokens + req.input_tokens + req.output_tokens,
                           dtype=torch.int64)
        token_idxs = torch.from_numpy(self.kv_cache.get_token_index([req]).astype(np.int64))
        shared = torch.tensor(req.shared_tokens, dtype=torch.int64)
        has_match_len = self.radix_cache.insert(key[:-1], token_idxs, shared)
        if has_match_len > len(req.shared_tokens):
            self.kv_cache.free_token_idxs(token_idxs[len(req.shared_tokens):has_match_len])
        self.kv_cache.free_rid(req.rid)
        return True

    def filter(self, req_ids):
        should_free_reqs = []
        for req_id in req_ids:
            if self.radix_cache is not None:
                self._free_req_cache(req_id)
            should_free_reqs.append(self.request_mapping.pop(req_id))
        last = [req.output_tokens[-1] for req in self.request_mapping.values()]
        self._refresh(False)
        self.is_prefill = False
        self.output_token_ids = torch.tensor(last, dtype=torch.int64, device=self.kv_cache.device)
        return should_free_reqs

    def update_forward_message(self, output_token_ids):
        """Record one generated token per request (one device->host read for
        the whole batch) and rebuild the decode metadata (runner_batch.py:227-243)."""
        self.is_prefill = False
        self.output_token_ids = output_token_ids.view(-1)
        toks = self.output_token_ids.tolist()
        req_ids = []
        for tok, req in zip(toks, self.request_mapping.values()):
            req_ids.append(req.id)
            req.update_forward_message(tok)
        self._refresh(False)
        return req_ids

    def update(self, new_runner_batch):
        """Merge another decode batch into this one (runner_batch.py:245-265)."""
        assert self.is_prefill is False and new_runner_batch.is_prefill is False, (
            "only decode batch can be merged")
        self.request_mapping.update(new_runner_batch.request_mapping)
        last = [req.output_tokens[-1] for req in self.request_mapping.values()]
        self._refresh(False)
        self.output_token_ids = torch.tensor(last, dtype=torch.int64, device=self.kv_cache.device)
        return True
