"""The scheduling loop (litelang/scheduler/scheduler.py:7-181)."""
from __future__ import annotations

import queue
import time

from .req_queue import ReadyQue, Req, ReqStatus, SchedulerRunnerQue, new_batch_id


class Scheduler:
    """Continuous batching over one model client.

    forward() is one scheduling round (scheduler.py:148-181): with no running
    batch, admit a new one, prefill it and decode up to 10 steps; with a
    running batch, admit, prefill and merge newcomers, then decode up to 10
    steps. Finished requests are filtered out of the model-side batch after
    every decode step; requests swapped out under KV pressure go back to the
    front of the ready queue with their generated tokens appended to the
    prompt."""

    def __init__(self, max_batch_size, tokenizer, max_total_length, max_output_length, max_reqs,
                 model_client, busy_scale, log=None):
        self.model_client_ = model_client
        max_sum_kv_tokens = self.model_client_.init_model()
        self.ready_and_swapped_que_ = ReadyQue(max_reqs, max_total_length - max_output_length,
                                               max_output_length, max_sum_kv_tokens,
                                               max_batch_size, busy_scale)
        self.running_que_ = SchedulerRunnerQue(max_batch_size, new_batch_id(), busy_scale,
                                               max_sum_kv_tokens)
        self.new_running_que_ = SchedulerRunnerQue(max_batch_size, new_batch_id(), busy_scale,
                                                   max_sum_kv_tokens)
        self.max_batch_size_ = max_batch_size
        self.tokenizer_ = tokenizer
        self.now_id = 0
        self.max_id = 100000
        self.max_total_length_ = max_total_length
        self.max_output_length_ = max_output_length
        self.now_decode_times_, self.every_decode_times_try_get_new_batch_ = 0, 10
        self.log_ = log  # optional callable(str): the reference prints throughput lines

    # ------------------------------------------------------------ requests
    def add_req(self, prompt, top_p, top_k, temperature, do_sample):
        # encode_single returns a batch of one sequence (tokenizer.py:15-24)
        toks = self.tokenizer_.encode_single(prompt)[0]
        toks = toks.tolist() if hasattr(toks, "tolist") else list(toks)
        return self.add_req_tokens(toks, top_p, top_k, temperature, do_sample, prompt=prompt)

    def add_req_tokens(self, input_tokens, top_p=1.0, top_k=1, temperature=0.0,
                       do_sample=False, prompt=""):
        """add_req for callers that already hold token ids."""
        toks = [int(t) for t in input_tokens]
        req = Req(id=self.now_id % self.max_id, status=ReqStatus.READY, prompt=prompt,
                  input_tokens=toks, output_tokens=[], max_total_length=self.max_total_length_,
                  max_output_length=self.max_output_length_, output_prompt_que=queue.Queue(),
                  top_p=top_p, top_k=top_k, temperature=temperature, do_sample=do_sample,
                  input_length=len(toks), eos_token=self.tokenizer_.eos_token_id)
        self.now_id += 1
        self.ready_and_swapped_que_.add_req(req)
        return req

    # ------------------------------------------------------------ batches
    def construct_running_que(self):
        self.running_que_ = self.ready_and_swapped_que_.try_generate_new_batch(self.running_que_)
        return True

    def try_construct_new_running_que(self):
        self.new_running_que_ = self.ready_and_swapped_que_.try_generate_new_batch(self.running_que_)

    def should_forward(self):
        return not self.running_que_.is_empty()

    def merge_runner_batch(self):
        self.model_client_.merge_batch(self.running_que_.batch_id, self.new_running_que_.batch_id)
        self.running_que_.update(self.new_running_que_)

    def _log(self, what, n, t0):
        if self.log_ is not None:
            self.log_(f"{what} throughput: {n / max(time.perf_counter() - t0, 1e-9)} tokens/s")

    def update_from_forward(self, output_token_ids, req_ids):
        texts = self.tokenizer_.decode(output_token_ids)
        return self.running_que_.update_from_forward(texts, output_token_ids, req_ids,
                                                     self.tokenizer_.eos_token_id)

    def model_prefill(self, batch_id):
        t0 = time.perf_counter()
        self.model_client_.add_batch(self.running_que_.get_transfer_data(), batch_id)
        toks, req_ids = self.model_client_.prefill(batch_id)
        self._filter_ended_at_prefill(batch_id, self.update_from_forward(toks, req_ids))
        self._log("prefill", len(req_ids), t0)
        return True

    def _filter_ended_at_prefill(self, batch_id, stop):
        # A request whose first token ends it leaves the scheduler's queue; the
        # reference leaves it in the model-side batch, where the next decode
        # returns an id the queue no longer holds (scheduler.py:97-103).
        # Here it is filtered out of the model-side batch as well.
        if stop:
            self.model_client_.filter_batch(batch_id, [r.id for r in stop])

    def model_decode(self, batch_id):
        t0 = time.perf_counter()
        swapped = self.running_que_.try_swapped_reqs()
        if swapped:
            self.model_client_.swapped_reqs(batch_id, [r.id for r in swapped])
            for r in swapped:
                r.input_tokens.extend(r.output_tokens)
                r.output_tokens = []
                r.is_prefill = True
                r.status = ReqStatus.SWAPPED
                self.ready_and_swapped_que_.add_swapped_req(r)
        toks, req_ids = self.model_client_.decode(batch_id)
        stop = self.update_from_forward(toks, req_ids)
        if stop:
            self.model_client_.filter_batch(batch_id, [r.id for r in stop])
        self._log("decode", len(req_ids), t0)
        return True

    def new_update_from_forward(self, output_token_ids, req_ids):
        texts = self.tokenizer_.decode(output_token_ids)
        return self.new_running_que_.update_from_forward(texts, output_token_ids, req_ids,
                                                         self.tokenizer_.eos_token_id)

    def new_model_prefill(self, batch_id):
        t0 = time.perf_counter()
        self.model_client_.add_batch(self.new_running_que_.get_transfer_data(), batch_id)
        toks, req_ids = self.model_client_.prefill(batch_id)
        self._filter_ended_at_prefill(batch_id, self.new_update_from_forward(toks, req_ids))
        self._log("prefill", len(req_ids), t0)
        return True

    def _decode_burst(self):
        while not self.running_que_.is_end():
            self.model_decode(self.running_que_.batch_id)
            self.now_decode_times_ += 1
            if self.now_decode_times_ >= self.every_decode_times_try_get_new_batch_:
                self.now_decode_times_ = 0
                break

    def forward(self):
        if self.running_que_.is_empty():
            self.construct_running_que()
            if self.running_que_.is_empty():
                return
            self.model_prefill(self.running_que_.batch_id)
            self._decode_burst()
        else:
            self.try_construct_new_running_que()
            if not self.new_running_que_.is_empty():
                self.new_model_prefill(self.new_running_que_.batch_id)
                self.merge_runner_batch()
            self._decode_burst()
        if self.running_que_.is_end():
            self.model_client_.remove_batch(self.running_que_.batch_id)
