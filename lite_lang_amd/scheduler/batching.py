"""The live batch and the waiting room of the continuous-batching scheduler.

Decision rules (the reference's, litelang/scheduler/req_queue.py:69-261,
restated; the recorded traces in tests/golden/scheduler_traces.json check that
every decision is the same):
  * admission takes waiting requests in order while the batch has room and the
    KV estimate still fits: with every forecast (held, expected) sorted by
    `expected` (descending, truncated to integers), the worst
    sum(held of the first j) + expected_j * j must stay within the KV budget;
  * the system counts as busy when the live batch's tokens (as of its last
    forward) plus those of the swapped-out requests exceed busy_scale x budget;
  * before a decode step that would exceed the budget, live requests are swapped
    out in the strategy's order until they free more than the excess; they go
    back to the front of the waiting queue.
"""
from __future__ import annotations

import uuid
from collections import deque
from typing import Dict, Iterable, List

import numpy as np

from .pause_strategy import STRATEGY_REGISTRY, select_swapped_reqs
from .request import Req, ReqStatus


def new_batch_id() -> str:
    return str(uuid.uuid4())


def estimate_fits(forecasts: Iterable, budget: int) -> bool:
    """Whether the KV estimate of `forecasts` ((held, expected) pairs) fits
    `budget` (req_queue.py:219-232). The order among equal `expected` values
    cannot change the result: within such a run the last prefix dominates."""
    rows = sorted(((int(h), int(e)) for h, e in forecasts), key=lambda r: r[1], reverse=True)
    held, worst = 0, None
    for rank, (h, e) in enumerate(rows, 1):
        held += h
        total = held + e * rank
        worst = total if worst is None else max(worst, total)
    return worst is None or worst <= budget


class LiveBatch:
    """The requests of one model-side batch and its KV bookkeeping."""

    def __init__(self, batch_id: str, kv_budget: int, swap_strategy: str = "LongestFirstStrategy"):
        self.batch_id = batch_id
        self.members: Dict[int, Req] = {}
        self.finished = False     # no request left after this batch's last forward
        self.kv_in_use = 0        # tokens held by the requests alive after that forward
        self._budget = kv_budget
        self._strategy = STRATEGY_REGISTRY[swap_strategy]()

    def __len__(self) -> int:
        return len(self.members)

    def empty(self) -> bool:
        return not self.members

    def add(self, req: Req) -> None:
        self.members[req.id] = req

    def transfer_data(self) -> List[dict]:
        """What the model side needs to build its batch."""
        return [{"id": r.id, "input_tokens": r.input_tokens, "temperature": r.temperature,
                 "top_p": r.top_p, "top_k": r.top_k, "do_sample": r.do_sample}
                for r in self.members.values()]

    def record(self, texts, tokens, req_ids) -> List[Req]:
        """Give every request of a forward its token; keep the unfinished ones
        (in the forward's order) and return the finished ones."""
        toks = np.asarray(tokens).reshape(len(req_ids), -1)[:, 0] if len(req_ids) else []
        alive: Dict[int, Req] = {}
        done: List[Req] = []
        for rid, text, tok in zip(req_ids, texts, toks):
            req = self.members[rid]
            if req.accept(text, tok):
                done.append(req)
            else:
                alive[rid] = req
        self.members = alive
        self.kv_in_use = sum(r.length for r in alive.values())
        self.finished = not alive
        return done

    def kv_excess(self) -> int:
        """Tokens by which the next forward would overrun the budget (<= 0: none)."""
        return self.kv_in_use + sum(r.step_tokens() for r in self.members.values()) - self._budget

    def swap_out_for_kv(self) -> List[Req]:
        """Remove and return the requests to swap out before the next step."""
        excess = self.kv_excess()
        if excess <= 0:
            return []
        victims = select_swapped_reqs(self.members.values(), self._strategy, excess)
        for r in victims:
            del self.members[r.id]
        return victims

    def absorb(self, other: "LiveBatch") -> None:
        """Merge a freshly prefilled batch into this one. Its KV count stays as
        of this batch's last forward until the next one."""
        self.members.update(other.members)
        self.finished = not self.members


class WaitingRoom:
    """Requests waiting for admission; swapped-out ones wait at the front."""

    def __init__(self, max_reqs: int, max_batch_size: int, kv_budget: int, busy_scale: float):
        self.max_reqs = max_reqs
        self.max_batch_size = max_batch_size
        self.kv_budget = kv_budget
        self.busy_threshold = kv_budget * busy_scale
        self.waiting: deque = deque()
        self.parked: deque = deque()  # swapped out and not yet re-admitted (newest first)

    def __len__(self) -> int:
        return len(self.waiting)

    def submit(self, req: Req) -> bool:
        """Queue a new request; refused (False) when max_reqs are already waiting."""
        if len(self.waiting) >= self.max_reqs:
            return False
        self.waiting.append(req)
        return True

    def return_swapped(self, req: Req) -> None:
        self.parked.appendleft(req)
        self.waiting.appendleft(req)

    def busy(self, live: LiveBatch) -> bool:
        return live.kv_in_use + sum(r.length for r in self.parked) > self.busy_threshold

    def admit(self, live: LiveBatch) -> LiveBatch:
        """A new batch of waiting requests that fit next to `live`."""
        fresh = LiveBatch(new_batch_id(), self.kv_budget)
        busy = self.busy(live)
        forecasts = [r.forecast(busy) for r in live.members.values()]
        size = len(live)
        while self.waiting and size < self.max_batch_size:
            head = self.waiting[0]
            assert head.status in (ReqStatus.READY, ReqStatus.SWAPPED), (
                f"request {head.id} waits in state {head.status}")
            cand = head.forecast(busy)
            if not estimate_fits(forecasts + [cand], self.kv_budget):
                break
            forecasts.append(cand)
            self.waiting.popleft()
            head.status = ReqStatus.RUNNER
            fresh.add(head)
            size += 1
        # re-admitted swapped requests leave the parked ledger (they were at
        # the front of the queue)
        for _ in range(min(len(fresh), len(self.parked))):
            self.parked.popleft()
        return fresh
