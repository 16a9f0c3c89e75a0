"""Request state and the two queues of the scheduler
(litelang/scheduler/req_queue.py:11-261)."""
from __future__ import annotations

import queue
import uuid
from collections import deque
from dataclasses import dataclass, field
from enum import Enum
from typing import List

import numpy as np

from .pause_strategy import STRATEGY_REGISTRY, select_swapped_reqs


def new_batch_id() -> str:
    return str(uuid.uuid4())


class ReqStatus(Enum):
    READY = 0
    RUNNER = 1
    SWAPPED = 2


@dataclass
class Req:
    """One request (req_queue.py:17-66)."""
    id: int
    status: ReqStatus
    prompt: str
    input_tokens: List[int]
    output_tokens: List[int]
    max_total_length: int
    max_output_length: int
    output_prompt_que: queue.Queue
    temperature: float
    top_p: float
    top_k: float
    do_sample: bool
    input_length: int
    eos_token: int
    is_prefill: bool = True
    output_length: int = 0
    is_end: bool = False

    def Add(self, text: str, output_token: int):
        """Record one generated token; the request ends on EOS, or once it is
        both at the total-length cap and at the output cap (:37-47)."""
        self.is_prefill = False
        self.output_length += 1
        if output_token == self.eos_token or (
                self.output_length + self.input_length >= self.max_total_length
                and self.output_length >= self.max_output_length):
            self.is_end = True
        self.output_prompt_que.put((text, self.is_end))
        self.output_tokens.append(int(output_token))

    @property
    def length(self):
        return self.input_length + self.output_length

    def next_forward_need_tokens(self):
        return self.input_length if self.is_prefill else 1

    def need_tokens(self, is_system_busy):
        """[tokens held now, tokens still expected] (:59-66): an idle system
        assumes 60% of the output cap until a request has produced that much."""
        held = self.input_length + self.output_length
        expect = self.max_output_length * (1 if is_system_busy else 0.6)
        if self.output_length >= expect:
            expect = self.max_output_length
        return [held, expect]


class SchedulerRunnerQue:
    """The requests of one model-side batch (req_queue.py:69-175)."""

    def __init__(self, max_batch_size, batch_id, busy_scale, max_sum_kv_tokens,
                 swapped_strategy="LongestFirstStrategy"):
        self.req_mappings = {}
        self.is_end_ = False
        self.is_prefill_ = False
        self.max_batch_size_ = max_batch_size
        self.busy_scale_ = busy_scale
        self.batch_id = batch_id
        self.has_been_consume_tokens = 0
        self.max_sum_kv_tokens_ = max_sum_kv_tokens
        self.strategy_ = STRATEGY_REGISTRY[swapped_strategy]()

    def add_req(self, req: Req):
        self.req_mappings[req.id] = req

    def req_count(self):
        return len(self.req_mappings)

    def update_from_forward(self, output_prompts, output_token_ids, req_ids, eos_token_id):
        """Append one token per request; returns the requests that ended.
        output_token_ids is host-side [B] or [B, 1]."""
        self.is_end_ = True
        self.is_prefill_ = False
        stop, remain, held = [], {}, 0
        toks = np.asarray(output_token_ids).reshape(len(req_ids), -1)[:, 0]
        for idx, text in enumerate(output_prompts):
            req = self.req_mappings[req_ids[idx]]
            req.Add(text, int(toks[idx]))
            if not req.is_end:
                self.is_end_ = False
                remain[req.id] = req
                held += req.length
            else:
                stop.append(req)
        self.has_been_consume_tokens = held
        self.req_mappings = remain
        return stop

    def is_end(self):
        return self.is_end_

    def is_empty(self):
        return len(self.req_mappings) == 0

    def get_transfer_data(self):
        return [{"id": r.id, "input_tokens": r.input_tokens, "temperature": r.temperature,
                 "top_p": r.top_p, "top_k": r.top_k, "do_sample": r.do_sample}
                for r in self.req_mappings.values()]

    def _next_forward_need_tokens(self):
        return sum(r.next_forward_need_tokens() for r in self.req_mappings.values())

    def can_decode(self):
        return self.has_been_consume_tokens + self._next_forward_need_tokens() - self.max_sum_kv_tokens_

    def try_swapped_reqs(self):
        """Swap out requests when the next step would exceed the KV budget."""
        need = self.has_been_consume_tokens + self._next_forward_need_tokens() - self.max_sum_kv_tokens_
        chosen = []
        if need > 0:
            chosen = select_swapped_reqs(self.req_mappings.values(), self.strategy_, need)
            for r in chosen:
                del self.req_mappings[r.id]
        return chosen

    def update(self, new_runner_batch):
        self.req_mappings.update(new_runner_batch.req_mappings)
        self.is_end_ = new_runner_batch.is_end_ | self.is_end_
        self.is_prefill_ = False
        return True

    @property
    def batch_size(self):
        return len(self.req_mappings)


class ReadyQue:
    """Waiting and swapped requests, and the admission rule (req_queue.py:178-261)."""

    def __init__(self, max_reqs, max_input_length, max_output_length, max_sum_kv_tokens,
                 max_batch_size, busy_scale):
        self.max_reqs_ = max_reqs
        self.max_input_length_ = max_input_length
        self.max_output_length_ = max_output_length
        self.max_sum_kv_tokens_ = max_sum_kv_tokens
        self.max_batch_size_ = max_batch_size
        self.busy_scale_ = busy_scale
        self.system_busy_threshold_ = self.max_sum_kv_tokens_ * self.busy_scale_
        self.reqs_ = deque()
        self.swapped_que_ = deque()
        self.cache_len_list_ = []

    def add_req(self, req: Req):
        if len(self.reqs_) >= self.max_reqs_:
            return False
        self.reqs_.append(req)
        return True

    def add_swapped_req(self, req: Req):
        self.swapped_que_.appendleft(req)
        self.reqs_.appendleft(req)
        return True

    def _is_system_busy(self, last_runner_batch):
        taken = last_runner_batch.has_been_consume_tokens + sum(r.length for r in self.swapped_que_)
        return taken > self.system_busy_threshold_

    def _can_add_new_req(self, new_req, is_system_busy):
        """Admit if, with requests ordered by expected remaining tokens
        (descending), the worst prefix estimate cumsum(held) + remaining * k
        stays within the KV budget (:219-232). The candidate stays in the
        estimate list whether or not it is admitted, as in the reference."""
        self.cache_len_list_.append(new_req.need_tokens(is_system_busy))
        need = np.array(self.cache_len_list_, dtype=np.int64)
        order = np.argsort(need[:, -1])[::-1]
        need = need[order]
        total = np.cumsum(need[:, 0]) + need[:, 1] * np.arange(1, need.shape[0] + 1)
        return int(np.max(total)) <= self.max_sum_kv_tokens_

    def try_generate_new_batch(self, last_runner_batch):
        new_batch = SchedulerRunnerQue(self.max_batch_size_, new_batch_id(), self.busy_scale_,
                                       self.max_sum_kv_tokens_)
        busy = self._is_system_busy(last_runner_batch)
        self.cache_len_list_ = [r.need_tokens(busy) for r in last_runner_batch.req_mappings.values()]
        size = last_runner_batch.batch_size
        while self.reqs_ and size < self.max_batch_size_:
            assert self.reqs_[0].status in (ReqStatus.READY, ReqStatus.SWAPPED), "bad request state"
            if not self._can_add_new_req(self.reqs_[0], busy):
                break
            req = self.reqs_.popleft()
            req.status = ReqStatus.RUNNER
            new_batch.add_req(req)
            size += 1
        for _ in range(min(new_batch.req_count(), len(self.swapped_que_))):
            self.swapped_que_.popleft()
        return new_batch
