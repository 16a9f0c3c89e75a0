"""Scheduler test workloads: a deterministic fake model side and scenarios.

FakeModelClient answers the scheduler's model calls like a model server that
generates token f(request id, tokens it has seen) and records every call, so
a scheduler's decisions (batch compositions, prefill/decode/merge/filter/swap
order, per-request outputs) become a comparable event list. Batch ids are
replaced by their order of first appearance. Used by make_scheduler_golden.py
(driving the reference scheduler) and by tests/test_scheduler.py (driving the
product); contains no scheduler logic.
"""
import numpy as np
import torch

EOS = 0


def token_of(rid, seen, mod=23):
    return (rid * 31 + seen * 17 + 5) % mod


class FakeTokenizer:
    eos_token_id = EOS

    def encode_single(self, prompt):
        return torch.tensor([[int(t) for t in prompt.split()]])

    def decode(self, token_ids):
        return [str(int(t)) for t in np.asarray(token_ids).reshape(-1)]


class FakeModelClient:
    def __init__(self, kv_tokens, as_tensor, mod=23):
        self.kv = kv_tokens
        self.mod = mod
        self.as_tensor = as_tensor  # the reference indexes rows of a tensor
        self.batches = {}
        self.events = []
        self.names = {}

    def _n(self, bid):
        if bid not in self.names:
            self.names[bid] = len(self.names)
        return self.names[bid]

    def init_model(self):
        return self.kv

    def add_batch(self, reqs, batch_id):
        self.batches[batch_id] = {r["id"]: len(r["input_tokens"]) for r in reqs}
        self.events.append(["add_batch", self._n(batch_id), [r["id"] for r in reqs],
                            [len(r["input_tokens"]) for r in reqs]])
        return True

    def _step(self, batch_id, what):
        b = self.batches[batch_id]
        ids = list(b.keys())
        toks = []
        for rid in ids:
            t = token_of(rid, b[rid], self.mod)
            if what == "prefill" and t == EOS:
                # the reference scheduler never filters a request that ends on
                # its first token (scheduler.py:97-103), so its next decode
                # would fail; recorded workloads avoid that case
                t = 1
            toks.append(t)
            b[rid] += 1
        self.events.append([what, self._n(batch_id), ids, toks])
        out = np.array(toks, dtype=np.int64).reshape(-1, 1)
        return (torch.from_numpy(out) if self.as_tensor else out), ids

    def prefill(self, batch_id):
        return self._step(batch_id, "prefill")

    def decode(self, batch_id):
        return self._step(batch_id, "decode")

    def filter_batch(self, batch_id, req_ids):
        for r in req_ids:
            del self.batches[batch_id][r]
        self.events.append(["filter", self._n(batch_id), list(req_ids)])
        return True

    def swapped_reqs(self, batch_id, req_ids):
        for r in req_ids:
            del self.batches[batch_id][r]
        self.events.append(["swapped", self._n(batch_id), list(req_ids)])
        return True

    def merge_batch(self, batch_id, new_batch_id):
        self.batches[batch_id].update(self.batches.pop(new_batch_id))
        self.events.append(["merge", self._n(batch_id), self._n(new_batch_id)])
        return True

    def remove_batch(self, batch_id):
        self.batches.pop(batch_id, None)
        self.events.append(["remove", self._n(batch_id)])
        return True


# (name, scheduler kwargs, kv tokens, prompt lengths, arrival schedule[, token modulus])
# arrivals: list of (round index, number of requests added before that round);
# a larger token modulus makes EOS rarer (longer generations, KV pressure)
SCENARIOS = [
    ("roomy", dict(max_batch_size=8, max_total_length=64, max_output_length=24, max_reqs=64, busy_scale=0.8),
     4096, [5, 9, 3, 12, 7, 4, 8, 10, 6, 11, 2, 13], [(0, 6), (2, 3), (5, 3)]),
    ("tight_kv", dict(max_batch_size=6, max_total_length=48, max_output_length=20, max_reqs=64, busy_scale=0.5),
     160, [9, 14, 6, 11, 8, 12, 7, 10, 13, 5, 9, 6, 15, 4], [(0, 8), (1, 2), (3, 4)]),
    ("swap_pressure", dict(max_batch_size=10, max_total_length=60, max_output_length=30, max_reqs=64, busy_scale=0.3),
     200, [12, 16, 10, 14, 18, 11, 13, 15, 9, 17, 12, 10], [(0, 10), (4, 2)]),
    ("small_batch", dict(max_batch_size=3, max_total_length=40, max_output_length=12, max_reqs=5, busy_scale=0.9),
     1000, [4, 6, 5, 7, 3, 8, 6, 5], [(0, 8)]),
    ("long_generations", dict(max_batch_size=8, max_total_length=120, max_output_length=100, max_reqs=64, busy_scale=0.95),
     300, [10, 20, 15, 25, 12, 18, 30, 8], [(0, 8), (3, 4)], 997),
    ("swap_then_readmit", dict(max_batch_size=6, max_total_length=90, max_output_length=70, max_reqs=64, busy_scale=0.99),
     220, [20, 30, 25, 15, 35, 10], [(0, 6), (6, 3)], 991),
]


def _has_work(sch):
    """A request is running or waiting (the product's Scheduler.has_work; the
    reference scheduler exposes only its queues)."""
    if hasattr(sch, "has_work"):
        return sch.has_work()
    return not sch.running_que_.is_empty() or bool(sch.ready_and_swapped_que_.reqs_)


def run(scheduler_cls, scenario, as_tensor, max_rounds=400):
    name, kw, kv, lens, arrivals = scenario[:5]
    mod = scenario[5] if len(scenario) > 5 else 23
    client = FakeModelClient(kv, as_tensor, mod)
    sch = scheduler_cls(kw["max_batch_size"], FakeTokenizer(), kw["max_total_length"],
                        kw["max_output_length"], kw["max_reqs"], client, kw["busy_scale"])
    reqs, nxt = [], 0
    arrivals = dict(arrivals)
    for rnd in range(max_rounds):
        for _ in range(arrivals.get(rnd, 0)):
            L = lens[nxt % len(lens)]
            prompt = " ".join(str(1 + (nxt * 7 + i) % 97) for i in range(L))
            reqs.append(sch.add_req(prompt, 1.0, 1, 0.0, False))
            nxt += 1
        if _has_work(sch) or rnd in arrivals:
            sch.forward()
        elif rnd > max(arrivals):
            break
    outputs = [[r.id, list(r.output_tokens), bool(r.is_end)] for r in reqs]
    return {"scenario": name, "events": client.events, "outputs": outputs}
