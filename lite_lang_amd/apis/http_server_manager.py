"""The scheduler behind the HTTP routes (counterpart of
litelang/apis/http_server_manager.py:10-58).

The reference builds its scheduler over rpyc model servers and lets the HTTP
threads call `Scheduler.add_req` while its loop thread runs `forward`. Here
the model side is in-process (`LocalModelClient`, one process per GPU), and
every scheduler call happens on the loop thread: an HTTP thread hands its
request to the loop through a queue and receives the queued `Req` back, then
reads the (text, is_end) pairs the scheduler puts on the request's
`output_prompt_que`. A request refused because `max_reqs` requests are
already waiting (which the reference leaves waiting forever) raises
`RequestRefused`; an exception in the loop thread is re-raised in every
generator that is waiting and in later calls.
"""
from __future__ import annotations

import os
import queue
import threading

from lite_lang_amd.scheduler import LocalModelClient, Scheduler

_IDLE_WAIT_S = 0.005  # how long an idle loop waits for a request before looking again


class RequestRefused(RuntimeError):
    """The waiting room is full (max_reqs requests already wait)."""


class HttpServerManager:
    def __init__(self, scheduler: Scheduler):
        self.scheduler_ = scheduler
        self._intake: queue.Queue = queue.Queue()
        self._stop = threading.Event()
        self._error: BaseException | None = None
        self._thread = threading.Thread(target=self.handle_loop, name="lite_lang_amd-scheduler",
                                        daemon=True)
        self._thread.start()

    @classmethod
    def from_model_path(cls, model_path, max_input_length, max_output_length, max_batch_size,
                        mem_usage, tp, max_reqs, busy_scale, use_radix_cache, tokenizer=None,
                        **runner_kwargs):
        """The reference constructor's arguments (http_server_manager.py:13-24):
        a Qwen2 checkpoint directory (config.json, safetensors or
        pytorch_model.bin, tokenizer files) served on this process's GPU."""
        from lite_lang_amd.models.qwen2 import Qwen2Config, Qwen2ModelRunner
        from lite_lang_amd.scheduler import Tokenizer
        if tp != 1:
            raise ValueError("this build serves one GPU per process (tp=1)")
        max_total_length = max_input_length + max_output_length
        config = Qwen2Config.from_json(os.path.join(model_path, "config.json"))
        runner = Qwen2ModelRunner(config.layer_nums, max_batch_size, config,
                                  max_length=max_total_length, model_path=model_path,
                                  mem_usage=mem_usage, use_radix_cache=use_radix_cache,
                                  **runner_kwargs)
        scheduler = Scheduler(max_batch_size=max_batch_size,
                              tokenizer=tokenizer if tokenizer is not None else Tokenizer(model_path),
                              max_total_length=max_total_length,
                              max_output_length=max_output_length, max_reqs=max_reqs,
                              model_client=LocalModelClient(runner), busy_scale=busy_scale)
        return cls(scheduler)

    # ------------------------------------------------------------ HTTP side
    def submit(self, prompt, top_p, top_k, temperature, do_sample):
        """Queue one request on the loop thread; returns its Req."""
        self._raise_if_failed()
        reply: queue.Queue = queue.Queue(maxsize=1)
        self._intake.put(((prompt, top_p, top_k, temperature, do_sample), reply))
        while True:
            try:
                req = reply.get(timeout=0.1)
            except queue.Empty:
                self._raise_if_failed()
                continue
            if isinstance(req, BaseException):
                raise req
            return req

    def generate(self, prompt, top_p, top_k, temperature, do_sample):
        """Yield the request's generated text piece by piece until it ends
        (http_server_manager.py:46-55)."""
        req = self.submit(prompt, top_p, top_k, temperature, do_sample)
        yield from self.stream(req)

    def stream(self, req):
        """The generated text of a submitted request, piece by piece."""
        while True:
            try:
                text, is_end = req.output_prompt_que.get(timeout=0.1)
            except queue.Empty:
                self._raise_if_failed()
                continue
            yield text
            if is_end:
                return

    # ------------------------------------------------------------ loop thread
    def handle_loop(self):
        try:
            while not self._stop.is_set():
                self._take_requests(block=not self.scheduler_.has_work())
                if self.scheduler_.has_work():
                    self.scheduler_.forward()
        except BaseException as e:  # surfaced to the HTTP side
            self._error = e

    def _take_requests(self, block):
        try:
            item = self._intake.get(timeout=_IDLE_WAIT_S) if block else self._intake.get_nowait()
        except queue.Empty:
            return
        while True:
            args, reply = item
            try:
                req = self.scheduler_.add_req(*args)
                reply.put(req if not req.refused else
                          RequestRefused("too many requests are waiting (max_reqs)"))
            except Exception as e:  # a bad prompt fails its own request only
                reply.put(e)
            try:
                item = self._intake.get_nowait()
            except queue.Empty:
                return

    def _raise_if_failed(self):
        if self._error is not None:
            raise RuntimeError("the scheduler loop stopped") from self._error

    def stop(self, timeout=10.0):
        """End the loop thread (requests still running get no more tokens)."""
        self._stop.set()
        self._thread.join(timeout)
