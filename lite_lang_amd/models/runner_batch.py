"""NoPad batch metadata and request bookkeeping.

Counterpart of litelang/models/runner_batch.py (get_no_padding_messages
:8-35, RunnerReq :38-85, RunnerBatch :88-265) with the same public API and
field names. Differences in mechanism, not in results:
  * the metadata lists are kept on the host and the device tensors
    (input_tokens, position_ids, b_start_idx, b_seq_len, b_shared_seq_len,
    b_rids) are built lazily, in one pinned upload, only when a forward that
    needs them reads them;
  * generated tokens are copied to a pinned host ring asynchronously; a
    request's `output_tokens` list is completed on first read (and at
    filter / merge / radix insert), so a decode loop does not wait on the
    device every step (the reference reads 2*B scalars per step,
    runner_batch.py:231-234);
  * a token id of -1 marks a decode step whose fused launch gave up a
    bounded flag wait (ll_argmax_status): reading one raises DecodeStepError
    instead of handing it to a request.
"""
from __future__ import annotations

from typing import Dict

import numpy as np
import torch

from .cache import PageCache
from .radix_cache import RadixTree


class DecodeStepError(RuntimeError):
    """A decode step returned token id -1: one of its fused launches gave up
    a bounded flag wait, so that step's outputs (and those of every later step
    until the error word is reset, Qwen2ModelRunner.reset_decode_fault) are
    invalid."""


def check_step_tokens(tokens, what="decode step"):
    """Raise DecodeStepError when any token id of a step is negative."""
    arr = np.asarray(tokens)
    if arr.size and int(arr.min()) < 0:
        raise DecodeStepError(
            f"{what}: token id -1 from the device: a fused decode launch gave up waiting on "
            "its producers (outputs of this step are invalid)")


def get_no_padding_messages_host(input_reqs, is_prefill=True):
    """Host lists (input_ids, position_ids, start_idx, seq_len, shared_len, rids)."""
    position_ids, input_ids, req_lengths, start_idx, shared_seq_len, rids = [], [], [], [], [], []
    for idx, req in enumerate(input_reqs):
        rids.append(req.rid)
        ns = len(req.shared_tokens)
        shared_seq_len.append(ns)
        if is_prefill:
            position_ids.extend(range(ns, ns + len(req.input_tokens)))
            start_idx.append(len(input_ids))
            input_ids.extend(req.input_tokens)
        else:
            position_ids.append(req.length - 1)
            start_idx.append(idx)
        req_lengths.append(req.length)
    return input_ids, position_ids, start_idx, req_lengths, shared_seq_len, rids


def _upload(lists, device):
    """One pinned host buffer -> device; returns int64 device tensors, one per list."""
    sizes = [len(x) for x in lists]
    flat = torch.empty(max(1, sum(sizes)), dtype=torch.int64, pin_memory=True)
    fn = flat.numpy()
    o = 0
    for x, n in zip(lists, sizes):
        fn[o:o + n] = x
        o += n
    dev = flat.to(device, non_blocking=True)
    out, o = [], 0
    for n in sizes:
        out.append(dev[o:o + n])
        o += n
    return out


def get_no_padding_messages(input_reqs, is_prefill=True, device="cuda"):
    """Device tensors (input_ids, position_ids, b_start_idx, b_seq_len,
    b_shared_seq_len, b_rids) as in runner_batch.py:8-35 (b_rids int32)."""
    h = get_no_padding_messages_host(input_reqs, is_prefill)
    t = _upload(list(h), device)
    return t[0], t[1], t[2], t[3], t[4], t[5].to(torch.int32)


class RunnerReq:
    """One admitted request (runner_batch.py:38-85)."""

    def __init__(self, id, rid, input_length, output_length=0, shared_tokens=None,
                 match_token_idxs=None, input_tokens=None, output_tokens=None,
                 temperature=0.0, top_p=0.0, top_k=0.0, do_sample=False):
        self.id, self.rid = id, rid
        self.input_length, self.output_length = input_length, output_length
        self.shared_tokens = shared_tokens if shared_tokens is not None else []
        self.match_token_idxs = match_token_idxs
        self.input_tokens = input_tokens
        self._output_tokens = output_tokens
        self.temperature, self.top_p, self.top_k, self.do_sample = temperature, top_p, top_k, do_sample
        self._batch = None  # batch holding not-yet-fetched tokens of this request

    @staticmethod
    def create_runner_req(id, input_tokens, shared_tokens, match_token_idxs, temperature, top_p,
                          top_k, do_sample) -> "RunnerReq":
        return RunnerReq(id=id, rid=None, input_length=len(input_tokens),
                         shared_tokens=shared_tokens, match_token_idxs=match_token_idxs,
                         input_tokens=input_tokens, temperature=temperature, top_p=top_p,
                         top_k=top_k, do_sample=do_sample)

    @property
    def output_tokens(self):
        if self._batch is not None:
            self._batch.flush()
        return self._output_tokens

    @output_tokens.setter
    def output_tokens(self, v):
        self._output_tokens = v

    @property
    def length(self):
        return len(self.shared_tokens) + self.input_length + self.output_length

    def update_forward_message(self, token_id):
        self.output_length += 1
        if self._output_tokens is None:
            self._output_tokens = []
        self._output_tokens.append(int(token_id))


class RunnerBatch:
    """A NoPad batch of admitted requests (runner_batch.py:88-265)."""

    TOKEN_RING = 64  # decode steps whose tokens may be in flight to the host

    def __init__(self, id, request_mapping: Dict[int, RunnerReq], is_prefill: bool,
                 radix_cache: RadixTree, kv_cache: PageCache):
        self.id = id
        self.request_mapping = request_mapping
        self.is_prefill = is_prefill
        self.radix_cache = radix_cache
        self.kv_cache = kv_cache
        self.output_token_ids = None
        self.host = None
        self._dev = None
        self._ring = None
        self._pending = []  # (ring row, requests, event), oldest first
        self._next_row = 0  # ring rows are used cyclically
        self._refresh_host()

    # ------------------------------------------------------------ metadata
    def _refresh_host(self):
        self.host = get_no_padding_messages_host(self.request_mapping.values(), self.is_prefill)
        self._dev = None

    def _device(self):
        if self._dev is None:
            t = _upload(list(self.host), self.kv_cache.device)
            self._dev = (t[0], t[1], t[2], t[3], t[4], t[5].to(torch.int32))
        return self._dev

    input_tokens = property(lambda self: self._device()[0])
    position_ids = property(lambda self: self._device()[1])
    b_start_idx = property(lambda self: self._device()[2])
    b_seq_len = property(lambda self: self._device()[3])
    b_shared_seq_len = property(lambda self: self._device()[4])
    b_rids = property(lambda self: self._device()[5])

    # ------------------------------------------------------------ admission
    @classmethod
    def create_batch(cls, req_messages, batch_id, is_prefill: bool = True, model_runner=None):
        """Admit requests (runner_batch.py:103-167): radix prefix match on all
        but the last prompt token, request-row allocation, shared-slot refs.

        Every prompt id is checked against the vocabulary first (nothing is
        admitted if one is out of range): the reference's torch.embedding
        raises on such an id at the forward, and the embedding kernel here
        would otherwise clamp it."""
        vocab = getattr(getattr(model_runner, "config_", None), "vocab_size", None)
        if vocab is not None:
            for message in req_messages:
                for t in message["input_tokens"]:
                    if not 0 <= int(t) < vocab:
                        raise ValueError(f"request {message['id']}: token id {int(t)} is outside "
                                         f"the vocabulary [0, {vocab})")
        request_mapping = {}
        for message in req_messages:
            request_id = message["id"]
            input_tokens = list(message["input_tokens"])
            shared_tokens = []
            match_token_idxs = None
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
        return cls(batch_id, request_mapping, is_prefill, model_runner.radix_cache,
                   model_runner.kv_cache)

    def get_post_sample_para(self):
        reqs = list(self.request_mapping.values())
        dev = self.kv_cache.device
        return (torch.tensor([r.temperature for r in reqs], device=dev),
                torch.tensor([r.top_p for r in reqs], device=dev),
                torch.tensor([r.top_k for r in reqs], device=dev),
                torch.tensor([r.do_sample for r in reqs], device=dev))

    # ------------------------------------------------------------ tokens
    def flush(self):
        """Complete every request's output_tokens with the fetched tokens."""
        if not self._pending:
            return
        self._pending[-1][2].synchronize()
        ring = self._ring.numpy()
        try:
            for row, reqs, _ in self._pending:
                check_step_tokens(ring[row, :len(reqs)])
        except DecodeStepError:
            self._pending = []  # the steps in flight are dropped with the error
            self._next_row = 0
            raise
        for row, reqs, _ in self._pending:
            for j, req in enumerate(reqs):
                if req._output_tokens is None:
                    req._output_tokens = []
                req._output_tokens.append(int(ring[row, j]))
                req._batch = None
        self._pending = []
        self._next_row = 0

    def _retire_oldest(self):
        """Hand the oldest in-flight step's tokens to its requests and free its
        ring row. That step finished long before the newest one, so this waits
        for nothing in steady state (flush() would drain the whole stream)."""
        row, reqs, ev = self._pending.pop(0)
        ev.synchronize()
        vals = self._ring[row].numpy()
        check_step_tokens(vals[:len(reqs)])
        for j, req in enumerate(reqs):
            if req._output_tokens is None:
                req._output_tokens = []
            req._output_tokens.append(int(vals[j]))

    def update_forward_message(self, output_token_ids):
        """Record one generated token per request and move to decode metadata
        (runner_batch.py:227-243). The tokens reach the host asynchronously."""
        self.is_prefill = False
        out = output_token_ids.view(-1)
        self.output_token_ids = out
        reqs = list(self.request_mapping.values())
        B = len(reqs)
        if self._ring is None or self._ring.shape[1] < B:
            self.flush()
            self._ring = torch.empty((self.TOKEN_RING, max(B, 1)), dtype=torch.int64,
                                     pin_memory=True)
        if len(self._pending) == self.TOKEN_RING:
            self._retire_oldest()
        row = self._next_row
        self._next_row = (row + 1) % self.TOKEN_RING
        self._ring[row, :B].copy_(out, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._pending.append((row, reqs, ev))
        req_ids = []
        for req in reqs:
            req.output_length += 1
            req._batch = self
            req_ids.append(req.id)
        self._refresh_host()
        return req_ids

    # ------------------------------------------------------------ membership
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
        """Drop finished requests (runner_batch.py:206-225)."""
        self.flush()
        should_free_reqs = []
        for req_id in req_ids:
            if self.radix_cache is not None:
                self._free_req_cache(req_id)
            should_free_reqs.append(self.request_mapping.pop(req_id))
        last = [req.output_tokens[-1] for req in self.request_mapping.values()]
        self.is_prefill = False
        self._refresh_host()
        self.output_token_ids = torch.tensor(last, dtype=torch.int64, device=self.kv_cache.device)
        return should_free_reqs

    def update(self, new_runner_batch):
        """Merge another decode batch into this one (runner_batch.py:245-265)."""
        assert self.is_prefill is False and new_runner_batch.is_prefill is False, (
            "only decode batch can be merged")
        self.flush()
        new_runner_batch.flush()
        self.request_mapping.update(new_runner_batch.request_mapping)
        last = [req.output_tokens[-1] for req in self.request_mapping.values()]
        self._refresh_host()
        self.output_token_ids = torch.tensor(last, dtype=torch.int64, device=self.kv_cache.device)
        return True
