"""A generation request and its KV-token accounting.

The fields are those the reference's front end and scheduler read
(litelang/scheduler/req_queue.py:17-34): the HTTP layer takes
(text, is_end) pairs from `output_prompt_que` (apis/http_server_manager.py:50-53).
The accounting rules are the reference's, restated:
  * a request ends on EOS, or once it holds max_total_length tokens *and*
    has produced max_output_length of them (req_queue.py:37-47);
  * the next forward stores input_length tokens for it if it must be
    (re)prefilled, else one (req_queue.py:53-57);
  * its forecast is (tokens held now, tokens it will still need): the output
    cap, scaled by 0.6 while the system is not busy and the request has
    produced less than that (req_queue.py:59-66).
input_length stays the original prompt length when a swapped-out request
gets its generated tokens appended to input_tokens (as in the reference), so
length keeps counting every token the request has produced.
"""
from __future__ import annotations

import queue
from dataclasses import dataclass
from enum import Enum
from typing import List

IDLE_OUTPUT_FRACTION = 0.6  # expected share of the output cap while the system is idle


class ReqStatus(Enum):
    READY = 0
    RUNNER = 1
    SWAPPED = 2


@dataclass
class Req:
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
    refused: bool = False  # not queued: max_reqs requests were already waiting

    @property
    def length(self) -> int:
        """Tokens the request holds in the KV cache once its last token is stored."""
        return self.input_length + self.output_length

    def accept(self, text: str, token: int) -> bool:
        """Take one generated token; publish it to the front end; return
        whether the request has finished."""
        token = int(token)
        self.is_prefill = False
        self.output_length += 1
        capped = (self.length >= self.max_total_length
                  and self.output_length >= self.max_output_length)
        if token == self.eos_token or capped:
            self.is_end = True
        self.output_prompt_que.put((text, self.is_end))
        self.output_tokens.append(token)
        return self.is_end

    def step_tokens(self) -> int:
        """KV tokens the next forward stores for this request."""
        return self.input_length if self.is_prefill else 1

    def forecast(self, busy: bool) -> tuple:
        """(tokens held, tokens still expected) for the admission estimate."""
        cap = self.max_output_length
        expected = cap if busy else cap * IDLE_OUTPUT_FRACTION
        if self.output_length >= expected:
            expected = cap
        return (self.length, expected)

    def park(self) -> None:
        """Swap out: fold the generated tokens into the prompt so a later
        prefill recomputes their KV, and wait for re-admission."""
        self.input_tokens.extend(self.output_tokens)
        self.output_tokens = []
        self.is_prefill = True
        self.status = ReqStatus.SWAPPED
