"""CPU restatement of the NoPad batch metadata (test infrastructure only).

Follows get_no_padding_messages, litelang/models/runner_batch.py:8-35, and
RunnerReq.length (runner_batch.py:77-79).
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class Req:
    rid: int
    input_tokens: list
    shared_tokens: list = field(default_factory=list)
    output_tokens: list = field(default_factory=list)

    @property
    def length(self) -> int:
        return len(self.shared_tokens) + len(self.input_tokens) + len(self.output_tokens)


def no_padding_messages(reqs, is_prefill: bool):
    """Returns (input_ids, position_ids, start_idx, seq_len, shared_len, rids).

    Prefill: positions shared+i of the non-shared tokens, starts = prefix sums
    of the input lengths. Decode: position length-1, start = batch index.
    seq_len is always the full request length.
    """
    input_ids, pos, start, lens, shared, rids = [], [], [], [], [], []
    for idx, r in enumerate(reqs):
        rids.append(r.rid)
        if is_prefill:
            shared.append(len(r.shared_tokens))
            pos.extend(i + len(r.shared_tokens) for i in range(len(r.input_tokens)))
            start.append(len(input_ids))
            input_ids.extend(r.input_tokens)
        else:
            pos.append(r.length - 1)
            start.append(idx)
        lens.append(r.length)
    return input_ids, pos, start, lens, shared, rids
