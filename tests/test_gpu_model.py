"""End-to-end parity of the Qwen2 runner on the GPU against the CPU oracle.

* BASELINE config 1 (tiny Qwen2, fp32, seed 0, 16-token prompt): the greedy
  tokens of 1 prefill + 31 decode steps must be identical to the oracle's.
* The same model in bf16 with a ragged 3-request batch: logits within
  max-abs 2e-2 of the bf16-emulating oracle for every step up to the first
  token divergence, and any divergence must be a near tie of the oracle.
Driven through the reference-shaped API: RunnerBatch.create_batch,
Qwen2ModelRunner.forward, RunnerBatch.update_forward_message
(test/generate_token.py:36-63).
"""
import pytest
import torch

from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle

pytestmark = pytest.mark.gpu


def _cfgs():
    from lite_lang_amd.models.qwen2.weights import tiny_config
    c = tiny_config()
    oc = Qwen2Cfg(num_layers=c.layer_nums, hidden=c.hidden_size, heads=c.num_heads,
                  kv_heads=c.num_key_value_heads, intermediate=c.intermediate_size,
                  vocab=c.vocab_size, tie_word_embeddings=c.tie_word_embeddings)
    return c, oc


def _run_product(cfg, sd, prompts, n_new, dtype, cuda, max_length=128):
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.runner_batch import RunnerBatch
    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, tp_rank=0, world_size=1, model_path=None,
                              max_length=max_length, mem_usage=0.5, use_radix_cache=False,
                              dtype=dtype, state_dict=sd, kv_max_size=1024, device=cuda)
    runner.init_model()
    msgs = [{"id": i, "input_tokens": list(p), "temperature": 0.0, "top_p": 1.0, "top_k": 1,
             "do_sample": False} for i, p in enumerate(prompts)]
    batch = RunnerBatch.create_batch(msgs, "b0", is_prefill=True, model_runner=runner)
    logits = []
    for _ in range(n_new):
        out = runner.forward(batch)
        logits.append(runner.model_ins_.last_logits.float().cpu())
        batch.update_forward_message(out)
    toks = torch.tensor([r.output_tokens for r in batch.request_mapping.values()])
    return toks, torch.stack(logits, 1)


def test_config1_fp32_greedy_tokens_identical(cuda):
    from lite_lang_amd.models.qwen2.weights import random_state_dict
    cfg, ocfg = _cfgs()
    sd = random_state_dict(cfg, seed=0)
    prompt = torch.randint(0, 1024, (16,), generator=torch.Generator().manual_seed(0)).tolist()
    print("case: config1 fp32 greedy 32", flush=True)
    ref = Qwen2Oracle(ocfg, sd, torch.float32, 8, 128, 1024).generate([prompt], 32)
    got, _ = _run_product(cfg, sd, [prompt], 32, torch.float32, cuda)
    assert got.tolist() == ref.tolist()


def test_tiny_bf16_ragged_batch_logits(cuda):
    from lite_lang_amd.models.qwen2.weights import random_state_dict
    cfg, ocfg = _cfgs()
    sd = random_state_dict(cfg, seed=1)
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in (16, 5, 40)]
    print("case: tiny bf16 ragged batch", flush=True)
    ref, ref_logits = Qwen2Oracle(ocfg, sd, torch.bfloat16, 8, 128, 1024).generate(
        prompts, 8, return_logits=True)
    got, got_logits = _run_product(cfg, sd, prompts, 8, torch.bfloat16, cuda)
    for b in range(len(prompts)):
        for s in range(8):
            d = float((got_logits[b, s].double() - ref_logits[b, s]).abs().max())
            assert d <= 2e-2, f"request {b} step {s}: logits max-abs {d}"
            if got[b, s] != ref[b, s]:
                top2 = ref_logits[b, s].topk(2).values
                assert float(top2[0] - top2[1]) <= 2e-2, "token divergence without a near tie"
                break
