"""In-process model side of the scheduler.

LocalModelClient offers the calls the reference's ModelServerRpc serves over
rpyc (litelang/scheduler/rpc/model_rpc.py:44-100) on a Qwen2ModelRunner in the
same process: one process drives one GPU, so there is no RPC hop and no
process group. Generated tokens are returned to the scheduler on the host
(one device-to-host read per step, as the reference's rpyc `obtain` does).
"""
from __future__ import annotations

import numpy as np

from lite_lang_amd.models.runner_batch import RunnerBatch, check_step_tokens


class IdTokenizer:
    """Stand-in tokenizer for token-id workloads (no tokenizer files are
    shipped): encode_single parses space-separated ids into a batch of one
    sequence, decode returns the ids as text, eos_token_id is configurable."""

    def __init__(self, eos_token_id=-1):
        self.eos_token_id = eos_token_id

    def encode_single(self, prompt):
        return [[int(t) for t in str(prompt).split()]]

    def decode(self, token_ids):
        return [str(int(t)) for t in np.asarray(token_ids).reshape(-1)]


class LocalModelClient:
    def __init__(self, model_runner):
        self.model_runner_ = model_runner
        self.batchs_ = {}

    def init_model(self):
        return self.model_runner_.init_model()

    def add_batch(self, req_messages, batch_id):
        self.batchs_[batch_id] = RunnerBatch.create_batch(req_messages, batch_id, is_prefill=True,
                                                          model_runner=self.model_runner_)
        return True

    def merge_batch(self, batch_id, new_batch_id):
        self.batchs_[batch_id].update(self.batchs_[new_batch_id])
        del self.batchs_[new_batch_id]
        return True

    def _step(self, batch_id):
        batch = self.batchs_[batch_id]
        out = self.model_runner_.forward(batch)
        req_ids = batch.update_forward_message(out)
        toks = out.view(-1, 1).cpu().numpy()
        check_step_tokens(toks)
        return toks, req_ids

    def prefill(self, batch_id):
        return self._step(batch_id)

    def decode(self, batch_id):
        return self._step(batch_id)

    def remove_batch(self, batch_id):
        if batch_id not in self.batchs_:
            return False
        self.model_runner_.free_reqs(self.batchs_[batch_id].request_mapping.values())
        del self.batchs_[batch_id]
        return True

    def filter_batch(self, batch_id, req_ids):
        self.model_runner_.free_reqs(self.batchs_[batch_id].filter(req_ids))
        return True

    def swapped_reqs(self, batch_id, req_ids):
        return self.filter_batch(batch_id, req_ids)
