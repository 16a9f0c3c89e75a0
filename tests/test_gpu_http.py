"""The HTTP front end over the real runner on the GPU (tiny fp32 Qwen2):
prompts posted to /generate and /generate_stream (in-process TestClient,
several at once) come back as the CPU oracle's greedy tokens
(litelang/apis/api_server.py routes over the scheduler)."""
import json
import threading

import pytest
import torch

from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle

pytestmark = pytest.mark.gpu


def test_http_generate_matches_oracle(cuda):
    from fastapi.testclient import TestClient
    from lite_lang_amd.apis import HttpServerManager, api_server
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import random_state_dict, tiny_config
    from lite_lang_amd.scheduler import IdTokenizer, LocalModelClient, Scheduler
    cfg = tiny_config()
    ocfg = Qwen2Cfg(num_layers=cfg.layer_nums, hidden=cfg.hidden_size, heads=cfg.num_heads,
                    kv_heads=cfg.num_key_value_heads, intermediate=cfg.intermediate_size,
                    vocab=cfg.vocab_size, tie_word_embeddings=cfg.tie_word_embeddings)
    sd = random_state_dict(cfg, seed=6)
    g = torch.Generator().manual_seed(6)
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in (9, 14, 5, 11)]
    max_out = 16
    print("case: http generate tiny fp32", flush=True)
    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, max_length=64, dtype=torch.float32,
                              state_dict=sd, device=cuda)
    sch = Scheduler(max_batch_size=4, tokenizer=IdTokenizer(eos_token_id=-1),
                    max_total_length=max_out + 1, max_output_length=max_out, max_reqs=32,
                    model_client=LocalModelClient(runner), busy_scale=0.9)
    m = HttpServerManager(sch)
    api_server.attach(m)
    try:
        client = TestClient(api_server.app)
        out = [None] * len(prompts)

        def one(i):
            body = {"prompt": " ".join(map(str, prompts[i]))}
            if i % 2:
                r = client.post("/generate_stream", json=body)
                out[i] = [int(json.loads(c)["generated_text"]) for c in r.text.split("\n\n") if c]
            else:
                out[i] = [int(t) for t in client.post("/generate", json=body).json()["result"]]

        ts = [threading.Thread(target=one, args=(i,)) for i in range(len(prompts))]
        for t in ts:
            t.start()
        for t in ts:
            t.join(120)
    finally:
        m.stop()
        api_server.attach(None)
    for i, p in enumerate(prompts):
        ref = Qwen2Oracle(ocfg, sd, torch.float32, 8, 64, 1024).generate([p], max_out)[0].tolist()
        assert out[i] == ref, f"prompt {i}"
