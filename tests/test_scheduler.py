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

from lite_lang_amd.scheduler import (STRATEGY_REGISTRY, LiveBatch, Req, ReqStatus,  # noqa: E402
                                     Scheduler, WaitingRoom, estimate_fits,
                                     select_swapped_reqs)

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
    sorted by expected remaining tokens, descending (req_queue.py:219-232);
    the expected counts are truncated to integers as the reference's int64
    array does."""
    new = _req(5, 40)  # idle system: expects 0.6 * 50 = 30 more
    assert new.forecast(False) == (40, 50 * 0.6)
    # sorted by remaining: (30, 50), (40, 30), (10, 20) -> 30+50*1, 70+30*2, 80+20*3 -> max 140
    rows = [(30, 50.0), (10, 20.0), new.forecast(False)]
    assert estimate_fits(rows, 140) and not estimate_fits(rows, 139)
    # truncation: 7 * 0.6 = 4.2 counts as 4 -> (10 + 4) = 14
    assert estimate_fits([(10, 4.2)], 14) and not estimate_fits([(10, 4.9)], 13)
    # equal expectations in any order give the same worst prefix
    a, b = [(5, 10), (30, 10), (1, 3)], [(30, 10), (5, 10), (1, 3)]
    assert estimate_fits(a, 55) and estimate_fits(b, 55) and not estimate_fits(a, 54)
    assert not estimate_fits(b, 54)
    # the waiting room admits in order while the estimate fits and the batch has room
    room = WaitingRoom(max_reqs=8, max_batch_size=3, kv_budget=140, busy_scale=0.8)
    live = LiveBatch("live", 140)
    for r in (_req(0, 30), _req(1, 40), _req(2, 40), _req(3, 10)):
        assert room.submit(r)
    fresh = room.admit(live)
    # 30+30 = 60; (30,30),(40,30): 70+60 = 130; a third (40, 30): 110+90 > 140
    assert list(fresh.members) == [0, 1] and len(room) == 2
    assert all(r.status == ReqStatus.RUNNER for r in fresh.members.values())


def test_need_tokens_and_end_rule():
    r = _req(1, 10, out=0, max_total=30, max_out=15)
    assert r.forecast(False) == (10, 15 * 0.6) and r.forecast(True) == (10, 15)
    r.output_length = 9
    assert r.forecast(False) == (19, 15)  # past 60% of the cap: assume the full cap
    r = _req(2, 10, max_total=20, max_out=15)
    for k in range(14):
        assert not r.accept("t", 7)  # total reached at 10 outputs, but output cap not yet
    assert r.accept("t", 7)
    assert r.is_end and r.output_length == 15
    assert [r.output_prompt_que.get()[1] for _ in range(15)] == [False] * 14 + [True]
    r = _req(3, 5)
    assert r.accept("t", 0) and r.is_end  # EOS


def test_swap_out_under_kv_pressure():
    """A live batch whose next step overruns the budget swaps out requests in
    the strategy's order until more than the excess is freed; they return to
    the front of the waiting queue with their tokens folded into the prompt."""
    live = LiveBatch("b", 100)
    reqs = [_req(i, n) for i, n in enumerate([30, 20, 40])]
    for r in reqs:
        r.is_prefill = False
        r.output_tokens = [9, 9]
        live.add(r)
    live.kv_in_use = 98  # + 3 new tokens -> 1 over
    assert live.kv_excess() == 1
    victims = live.swap_out_for_kv()
    assert [v.id for v in victims] == [1]  # shortest first under LongestFirstStrategy
    room = WaitingRoom(8, 4, 100, 0.5)
    room.submit(_req(7, 5))
    victims[0].park()
    room.return_swapped(victims[0])
    assert [r.id for r in room.waiting] == [1, 7] and victims[0].status == ReqStatus.SWAPPED
    assert victims[0].input_tokens == [1] * 20 + [9, 9] and victims[0].is_prefill


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
