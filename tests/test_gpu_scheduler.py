"""The scheduler driving the real runner on the GPU (tiny fp32 Qwen2).

Requests arrive in two waves through Scheduler -> LocalModelClient ->
Qwen2ModelRunner, so the run admits, prefills, merges, decodes in bursts and
filters finished requests (scheduler.py:148-181); the KV budget is small
enough that the scheduler swaps requests out and later re-prefills them with
their generated tokens appended (scheduler.py:107-121). Every request's full
generation must equal the CPU oracle's greedy generation for its prompt.
"""
import pytest
import torch

from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle

pytestmark = pytest.mark.gpu


def test_scheduler_end_to_end_with_swaps(cuda):
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import random_state_dict, tiny_config
    from lite_lang_amd.scheduler import IdTokenizer, LocalModelClient, Scheduler
    cfg = tiny_config()
    ocfg = Qwen2Cfg(num_layers=cfg.layer_nums, hidden=cfg.hidden_size, heads=cfg.num_heads,
                    kv_heads=cfg.num_key_value_heads, intermediate=cfg.intermediate_size,
                    vocab=cfg.vocab_size, tie_word_embeddings=cfg.tie_word_embeddings)
    sd = random_state_dict(cfg, seed=4)
    g = torch.Generator().manual_seed(4)
    lens = [12, 20, 7, 16, 9, 25]
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in lens]
    max_out = 24
    print("case: scheduler e2e tiny fp32 with swaps", flush=True)
    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, max_length=128, dtype=torch.float32,
                              state_dict=sd, kv_max_size=150, device=cuda)
    sch = Scheduler(max_batch_size=4, tokenizer=IdTokenizer(eos_token_id=-1),
                    max_total_length=max_out + 1, max_output_length=max_out, max_reqs=32,
                    model_client=LocalModelClient(runner), busy_scale=0.9)
    reqs = [sch.add_req_tokens(p) for p in prompts[:4]]
    rounds = 0
    swaps = 0
    orig_swap = sch.client.swapped_reqs

    def count_swaps(bid, ids):
        nonlocal swaps
        swaps += len(ids)
        return orig_swap(bid, ids)
    sch.client.swapped_reqs = count_swaps
    while rounds < 200 and (not all(r.is_end for r in reqs) or len(reqs) < len(prompts)):
        if rounds == 3:
            reqs += [sch.add_req_tokens(p) for p in prompts[4:]]
        sch.forward()
        rounds += 1
    assert all(r.is_end for r in reqs)
    assert swaps > 0, "the KV budget should have forced a swap-out"
    for r, p in zip(reqs, prompts):
        full = r.input_tokens[len(p):] + r.output_tokens  # swapped requests carry their tokens in the prompt
        assert r.output_length == max_out
        ref = Qwen2Oracle(ocfg, sd, torch.float32, 8, 128, 1024).generate([p], max_out)[0].tolist()
        assert full == ref, f"request {r.id}"
