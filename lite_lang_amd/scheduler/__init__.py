"""Continuous-batching scheduler of the Qwen2 token loop (host side).

Counterpart of litelang/scheduler/{scheduler.py, req_queue.py,
pause_strategy.py}: admission by the estimated KV-token budget, decode bursts
of 10 steps between admissions, merging of newly prefilled batches into the
running one, swap-out under KV pressure. The model side is in-process
(model_client.LocalModelClient) instead of the reference's rpyc workers: one
process drives one GPU.
"""
from .pause_strategy import STRATEGY_REGISTRY, select_swapped_reqs
from .request import Req, ReqStatus
from .batching import LiveBatch, WaitingRoom, estimate_fits
from .scheduler import Scheduler
from .model_client import LocalModelClient, IdTokenizer
from .tokenizer import Tokenizer

__all__ = ["Scheduler", "Req", "ReqStatus", "LiveBatch", "WaitingRoom", "estimate_fits",
           "STRATEGY_REGISTRY", "select_swapped_reqs", "LocalModelClient", "IdTokenizer",
           "Tokenizer"]
