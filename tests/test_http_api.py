"""The HTTP front end (lite_lang_amd/apis, counterpart of litelang/apis/) on
the CPU: the FastAPI routes driven in-process (fastapi's TestClient) over
the real Scheduler and HttpServerManager, with a deterministic fake model
side whose next token depends only on the request's prompt and how many
tokens it has produced, so every response can be predicted exactly.
Checked: /generate and /generate_stream return the same pieces, in order,
as the scheduler run directly; concurrent requests each get their own
tokens; a full waiting room answers 503; an error in the model side reaches
the waiting request instead of hanging it.
"""
import json
import threading

import numpy as np
import pytest

fastapi = pytest.importorskip("fastapi")
from fastapi.testclient import TestClient  # noqa: E402

from lite_lang_amd.apis import HttpServerManager, api_server  # noqa: E402
from lite_lang_amd.scheduler import IdTokenizer, Scheduler  # noqa: E402

MAX_OUT, MAX_TOTAL = 9, 16


def next_token(prompt, n_out):
    return (sum(prompt) * 7 + n_out * 13) % 97 + 1  # never 0 (the tokenizer's EOS below)


class PromptModel:
    """Model side of the scheduler: token k of a request is next_token(prompt, k)."""

    def __init__(self, kv_tokens=4096, fail=False):
        self.kv = kv_tokens
        self.fail = fail
        self.batches = {}

    def init_model(self):
        return self.kv

    def add_batch(self, reqs, batch_id):
        self.batches[batch_id] = {r["id"]: [list(r["input_tokens"]), 0] for r in reqs}
        return True

    def _step(self, batch_id):
        if self.fail:
            raise RuntimeError("model side failed")
        b = self.batches[batch_id]
        ids = list(b.keys())
        toks = []
        for rid in ids:
            prompt, n = b[rid]
            toks.append(next_token(prompt, n))
            b[rid][1] = n + 1
        return np.array(toks, dtype=np.int64).reshape(-1, 1), ids

    prefill = _step
    decode = _step

    def filter_batch(self, batch_id, req_ids):
        for r in req_ids:
            del self.batches[batch_id][r]
        return True

    swapped_reqs = filter_batch

    def merge_batch(self, batch_id, new_batch_id):
        self.batches[batch_id].update(self.batches.pop(new_batch_id))
        return True

    def remove_batch(self, batch_id):
        self.batches.pop(batch_id, None)
        return True


def expected(prompt):
    """A request ends once it holds MAX_TOTAL tokens and has produced MAX_OUT
    (req_queue.py:37-47; no EOS here)."""
    n = max(MAX_OUT, MAX_TOTAL - len(prompt))
    return [str(next_token(prompt, k)) for k in range(n)]


@pytest.fixture
def server():
    made = []

    def make(max_reqs=64, fail=False):
        sch = Scheduler(max_batch_size=4, tokenizer=IdTokenizer(eos_token_id=0),
                        max_total_length=MAX_TOTAL, max_output_length=MAX_OUT, max_reqs=max_reqs,
                        model_client=PromptModel(fail=fail), busy_scale=0.8)
        m = HttpServerManager(sch)
        made.append(m)
        api_server.attach(m)
        return TestClient(api_server.app), m
    yield make
    for m in made:
        m.stop()
    api_server.attach(None)


def test_generate_returns_every_piece(server):
    client, _ = server()
    r = client.post("/generate", json={"prompt": "3 5 7"})
    assert r.status_code == 200
    assert r.json() == {"result": expected([3, 5, 7])}


def test_generate_stream_chunks(server):
    client, _ = server()
    r = client.post("/generate_stream", json={"prompt": "11 2", "top_k": 1})
    assert r.status_code == 200
    assert r.headers["content-type"].startswith("text/event-stream")
    chunks = [c for c in r.text.split("\n\n") if c]
    assert [json.loads(c)["generated_text"] for c in chunks] == expected([11, 2])


def test_concurrent_requests_get_their_own_tokens(server):
    client, _ = server()
    prompts = [[i, i + 1, 2 * i] for i in range(1, 11)]
    out = [None] * len(prompts)

    def one(i):
        out[i] = client.post("/generate", json={"prompt": " ".join(map(str, prompts[i]))}).json()

    ts = [threading.Thread(target=one, args=(i,)) for i in range(len(prompts))]
    for t in ts:
        t.start()
    for t in ts:
        t.join(30)
    assert [o["result"] for o in out] == [expected(p) for p in prompts]


def test_manager_generator_matches_the_reference_shape(server):
    _, m = server()
    assert list(m.generate("4 4", 1.0, 1, 1.0, False)) == expected([4, 4])


def test_full_waiting_room_answers_503(server):
    client, _ = server(max_reqs=0)
    r = client.post("/generate", json={"prompt": "1 2"})
    assert r.status_code == 503


def test_model_failure_reaches_the_request(server):
    client, m = server(fail=True)
    with pytest.raises(RuntimeError, match="scheduler loop stopped"):
        list(m.generate("1 2", 1.0, 1, 1.0, False))
    # the HTTP route reports it as a server error instead of hanging
    client2 = TestClient(api_server.app, raise_server_exceptions=False)
    assert client2.post("/generate", json={"prompt": "3"}).status_code == 500
