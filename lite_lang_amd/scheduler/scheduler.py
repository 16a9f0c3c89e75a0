"""The continuous-batching loop (counterpart of litelang/scheduler/scheduler.py:7-181).

One `forward()` is one scheduling round: admit a batch from the waiting room
(prefill it, and merge it into the live batch if one is running), then decode
the live batch for at most BURST_STEPS steps before the next admission
attempt. The burst counter carries over between rounds (a batch that ends
early leaves the rest of the burst to the next one), as in the reference.
The model side is any object with the reference ModelClient's calls
(init_model, add_batch, prefill, decode, merge_batch, filter_batch,
swapped_reqs, remove_batch); LocalModelClient serves them in-process.
"""
from __future__ import annotations

import queue
import time

from .batching import LiveBatch, WaitingRoom, new_batch_id
from .request import Req, ReqStatus

MAX_REQUEST_ID = 100000  # request ids wrap at this value (scheduler.py:40)


class Scheduler:
    BURST_STEPS = 10

    def __init__(self, max_batch_size, tokenizer, max_total_length, max_output_length, max_reqs,
                 model_client, busy_scale, log=None):
        self.client = model_client
        self.tokenizer = tokenizer
        self.max_batch_size = max_batch_size
        self.max_total_length = max_total_length
        self.max_output_length = max_output_length
        kv_budget = self.client.init_model()
        self._room = WaitingRoom(max_reqs, max_batch_size, kv_budget, busy_scale)
        self._kv_budget = kv_budget
        self._live = LiveBatch(new_batch_id(), kv_budget)
        self._burst = 0
        self._submitted = 0
        self._log = log  # optional callable(str) for throughput lines (the reference prints them)

    # ------------------------------------------------------------ requests
    def add_req(self, prompt, top_p, top_k, temperature, do_sample) -> Req:
        """Tokenise `prompt` and queue it; the caller reads the generated text
        from the returned request's output_prompt_que."""
        ids = self.tokenizer.encode_single(prompt)[0]  # a batch of one sequence
        ids = ids.tolist() if hasattr(ids, "tolist") else list(ids)
        return self.add_req_tokens(ids, top_p, top_k, temperature, do_sample, prompt=prompt)

    def add_req_tokens(self, input_tokens, top_p=1.0, top_k=1, temperature=0.0, do_sample=False,
                       prompt="") -> Req:
        """add_req for callers that already hold token ids. A request arriving
        while max_reqs are waiting is not queued (it never runs), as in the
        reference; its `refused` flag tells the caller."""
        toks = [int(t) for t in input_tokens]
        req = Req(id=self._submitted % MAX_REQUEST_ID, status=ReqStatus.READY, prompt=prompt,
                  input_tokens=toks, output_tokens=[], max_total_length=self.max_total_length,
                  max_output_length=self.max_output_length, output_prompt_que=queue.Queue(),
                  temperature=temperature, top_p=top_p, top_k=top_k, do_sample=do_sample,
                  input_length=len(toks), eos_token=self.tokenizer.eos_token_id)
        self._submitted += 1
        req.refused = not self._room.submit(req)
        return req

    def has_work(self) -> bool:
        """Whether a request is running or waiting."""
        return not self._live.empty() or len(self._room) > 0

    # ------------------------------------------------------------ one round
    def forward(self) -> None:
        if self._live.empty():
            self._live = self._room.admit(self._live)
            if self._live.empty():
                return
            self._prefill(self._live)
        else:
            fresh = self._room.admit(self._live)
            if not fresh.empty():
                self._prefill(fresh)
                self.client.merge_batch(self._live.batch_id, fresh.batch_id)
                self._live.absorb(fresh)
        while not self._live.finished:
            self._decode_step()
            self._burst += 1
            if self._burst >= self.BURST_STEPS:
                self._burst = 0
                break
        if self._live.finished:
            self.client.remove_batch(self._live.batch_id)

    # ------------------------------------------------------------ model calls
    def _apply(self, batch: LiveBatch, tokens, req_ids):
        """Hand a forward's tokens to the batch; drop finished requests from the
        model-side batch. (A request that ends on its prefill token is dropped
        too: the reference leaves it in the model-side batch, where its next
        decode hands back an id the scheduler no longer holds,
        scheduler.py:97-103.)"""
        done = batch.record(self.tokenizer.decode(tokens), tokens, req_ids)
        if done:
            self.client.filter_batch(batch.batch_id, [r.id for r in done])

    def _prefill(self, batch: LiveBatch) -> None:
        t0 = time.perf_counter()
        self.client.add_batch(batch.transfer_data(), batch.batch_id)
        tokens, req_ids = self.client.prefill(batch.batch_id)
        self._apply(batch, tokens, req_ids)
        self._report("prefill", len(req_ids), t0)

    def _decode_step(self) -> None:
        t0 = time.perf_counter()
        live = self._live
        victims = live.swap_out_for_kv()
        if victims:
            self.client.swapped_reqs(live.batch_id, [r.id for r in victims])
            for r in victims:
                r.park()
                self._room.return_swapped(r)
        tokens, req_ids = self.client.decode(live.batch_id)
        self._apply(live, tokens, req_ids)
        self._report("decode", len(req_ids), t0)

    def _report(self, what, n, t0):
        if self._log is not None:
            self._log(f"{what} throughput: {n / max(time.perf_counter() - t0, 1e-9)} tokens/s")
