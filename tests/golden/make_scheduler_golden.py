"""Writes tests/golden/scheduler_traces.json: the reference scheduler's
decisions (litelang/scheduler/scheduler.py, req_queue.py, pause_strategy.py)
on the workloads of sched_scenarios.py, recorded by running those modules in
the build container (pure Python; no model, GPU or RPC is involved: the model
side is sched_scenarios.FakeModelClient). Run from the repository root:
    python tests/golden/make_scheduler_golden.py
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, "/root/reference")

import sched_scenarios  # noqa: E402
from litelang.scheduler.scheduler import Scheduler  # noqa: E402


def main():
    traces = [sched_scenarios.run(Scheduler, sc, as_tensor=True) for sc in sched_scenarios.SCENARIOS]
    out = os.path.join(HERE, "scheduler_traces.json")
    json.dump({"source": "litelang/scheduler/{scheduler,req_queue,pause_strategy}.py",
               "generator": os.path.basename(__file__), "traces": traces}, open(out, "w"))
    print(f"wrote {out}: " + ", ".join(f"{t['scenario']} {len(t['events'])} events" for t in traces))


if __name__ == "__main__":
    main()
