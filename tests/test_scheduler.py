"""Continuous-batching scheduler (litelang/scheduler/*) on the CPU.

The product scheduler must take exactly the reference's decisions: the
recorded traces (tests/golden/scheduler_traces.json, written by
tests/golden/make_scheduler_golden.py from the reference modules) list every
model-side call -- batch compositions, prefill/decode order, merges, filters,
swap-outs -- and every request's generated tokens; replaying the same
workloads on the product must give the same lists. Plus closed-form checks of
the admission estimate, the swap selection and the end-of-request rule.
"""
import json
import os
import queue
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import sched_scenarios  # noqa: E402

from lite_lang_amd.scheduler import (STRATEGY_REGISTRY, ReadyQue, Req, ReqStatus,  # noqa: E402
                                     Scheduler, SchedulerRunnerQue, select_swapped_reqs)

GOLD = os.path.join(os.path.dirname(__file__), "golden", "scheduler_traces.json")


def _traces():
    return {t["scenario"]: t for t in json.load(open(GOLD))["traces"]}


@pytest.mark.parametrize("scenario", sched_scenarios.SCENARIOS, ids=lambda s: s[0])
def test_decisions_equal_reference_traces(scenario):
    ref = _traces()[scenario[0]]
    got = sched_scenarios.run(Scheduler, scenario, as_tensor=False)
    for i, (a, b) in enumerate(zip(got["events"], ref["events"])):
        assert a == b, f"{scenario[0]}: event {i}: {a} != {b}"
    assert len(got["events"]) == len(ref["events"])
    assert got["outputs"] == ref["outputs"]


def test_traces_cover_merges_and_swaps():
    kinds = {e[0] for t in _traces().values() for e in t["events"]}
    assert {"add_batch", "prefill", "decode", "filter", "merge", "swapped", "remove"} <= kinds


def _req(i, inp, out=0, max_total=100, max_out=50):
    r = Req(id=i, status=ReqStatus.READY, prompt="", input_tokens=[1] * inp, output_tokens=[],
            max_total_length=max_total, max_output_length=max_out, output_prompt_que=queue.Queue(),
            temperature=0.0, top_p=1.0, top_k=1, do_sample=False, input_length=inp, eos_token=0)
    r.output_length = out
    return r


def test_admission_estimate_closed_form():
    """Admit iff max_j (sum_{i<=j} held_i + rem_j * j) <= budget over requests
    sorted by expected remaining tokens, descending (req_queue.py:219-232)."""
    rq = ReadyQue(64, 100, 50, 1000, 8, 0.8)
    rq.cache_len_list_ = [[30, 50.0], [10, 20.0]]
    new = _req(5, 40)  # idle system: expects 0.6 * 50 = 30 more
    # sorted by remaining: (30, 50), (40, 30), (10, 20) -> 30+50*1, 70+30*2, 80+20*3 -> max 140
    assert rq._can_add_new_req(new, False)
    rq2 = ReadyQue(64, 100, 50, 139, 8, 0.8)
    rq2.cache_len_list_ = [[30, 50.0], [10, 20.0]]
    assert not rq2._can_add_new_req(new, False)


def test_need_tokens_and_end_rule():
    r = _req(1, 10, out=0, max_total=30, max_out=15)
    assert r.need_tokens(False) == [10, 15 * 0.6] and r.need_tokens(True) == [10, 15]
    r.output_length = 9
    assert r.need_tokens(False) == [19, 15]  # past 60% of the cap: assume the full cap
    r = _req(2, 10, max_total=20, max_out=15)
    for k in range(14):
        r.Add("t", 7)
        assert not r.is_end  # total reached at 10 outputs, but output cap not yet
    r.Add("t", 7)
    assert r.is_end and r.output_length == 15
    r = _req(3, 5)
    r.Add("t", 0)
    assert r.is_end  # EOS


def test_swap_selection_strategies():
    reqs = [_req(i, inp) for i, inp in enumerate([30, 10, 50, 20])]
    # LongestFirstStrategy orders by ascending length (pause_strategy.py:34-37)
    got = select_swapped_reqs(reqs, STRATEGY_REGISTRY["LongestFirstStrategy"](), 25)
    assert [r.id for r in got] == [1, 3]  # 10 + 20 > 25
    got = select_swapped_reqs(reqs, STRATEGY_REGISTRY["FIFOStrategy"](), 30)
    assert [r.id for r in got] == [0, 1]  # 30, then 40 > 30
    got = select_swapped_reqs(reqs, STRATEGY_REGISTRY["LIFOStrategy"](), 5)
    assert [r.id for r in got] == [3]


def test_first_token_eos_is_filtered():
    """Deviation from the reference (which fails on the next decode): a request
    ending on its first token leaves the model-side batch at once."""
    class EosFirst(sched_scenarios.FakeModelClient):
        def _step(self, batch_id, what):
            out, ids = super()._step(batch_id, what)
            if what == "prefill":
                out[0, 0] = sched_scenarios.EOS
                self.events[-1][3][0] = sched_scenarios.EOS
            return out, ids
    client = EosFirst(4096, False)
    sch = Scheduler(4, sched_scenarios.FakeTokenizer(), 40, 10, 16, client, 0.8)
    reqs = [sch.add_req("3 4 5", 1.0, 1, 0.0, False) for _ in range(3)]
    for _ in range(10):
        sch.forward()
    assert reqs[0].is_end and reqs[0].output_tokens == [sched_scenarios.EOS]
    assert ["filter", 0, [0]] in client.events
    assert all(r.is_end for r in reqs)
