"""SmoothQuant checkpoint ingestion on the GPU: the converter's output
(tests/hf_tiny.py:make_smoothquant_checkpoint; int8 weights, fp16
weight_scale, static quant_scale on o_proj/down_proj, pytorch_model.bin)
loaded through model_path -- the runner detects the int8 checkpoint and runs
its W8A8 runtime -- against the CPU oracle reading the same files.

Bars as for the W8A8 runtime on float checkpoints: fp32 storage gives the
oracle's greedy tokens exactly (the int32 products are exact and the
dequantisation is evaluated in the same fp32 order); fp16 storage, the
checkpoint's own dtype, is held to max-abs 4e-2 on the logits of a prefill
and decode steps (a single activation rounding can flip across a
quantisation step, the same bar as the bf16 W8A8 model test). Both the
static quantiser (quant_scale) and the per-token one run in every layer.
"""
import pytest
import torch

from tests.hf_tiny import corpus, make_checkpoint, make_smoothquant_checkpoint

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    from transformers import AutoTokenizer
    d = str(tmp_path_factory.mktemp("qwen2_tiny_float_gpu"))
    hf = make_checkpoint(d, seed=0)
    tok = AutoTokenizer.from_pretrained(d, local_files_only=True)
    sq = str(tmp_path_factory.mktemp("qwen2_tiny_sq_gpu"))
    sd = make_smoothquant_checkpoint(sq, hf, [tok(t)["input_ids"] for t in corpus(8, seed=3)])
    prompts = [tok(t)["input_ids"] for t in corpus(3, seed=7)]
    return sq, sd, prompts


def _product(sq, prompts, n_new, dtype, cuda, graph):
    import os
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import Qwen2Config
    from lite_lang_amd.models.runner_batch import RunnerBatch
    cfg = Qwen2Config.from_json(os.path.join(sq, "config.json"))
    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, model_path=sq, max_length=128, dtype=dtype,
                              kv_max_size=1024, device=cuda, use_cuda_graph=graph)
    runner.init_model()
    assert runner.model_ins_.quant == "w8a8"
    msgs = [{"id": i, "input_tokens": list(p), "temperature": 0.0, "top_p": 1.0, "top_k": 1,
             "do_sample": False} for i, p in enumerate(prompts)]
    batch = RunnerBatch.create_batch(msgs, "sq", is_prefill=True, model_runner=runner)
    logits = []
    for _ in range(n_new):
        out = runner.forward(batch)
        logits.append(runner.model_ins_.last_logits.float().cpu())
        batch.update_forward_message(out)
    toks = torch.tensor([r.output_tokens for r in batch.request_mapping.values()])
    return toks, torch.stack(logits, 1)


def _oracle(sd, prompts, n_new, dtype):
    from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle
    oc = Qwen2Cfg(num_layers=2, hidden=256, heads=4, kv_heads=2, intermediate=688, vocab=1024)
    return Qwen2Oracle(oc, sd, dtype, 8, 128, 1024, quant="w8a8").generate(
        prompts, n_new, return_logits=True)


@pytest.mark.parametrize("graph", [True, False])
def test_int8_checkpoint_fp32_tokens_identical(cuda, ckpt, graph):
    sq, sd, prompts = ckpt
    print(f"case: SmoothQuant checkpoint fp32 graph={graph}", flush=True)
    got, _ = _product(sq, prompts, 10, torch.float32, cuda, graph)
    ref, _ = _oracle(sd, prompts, 10, torch.float32)
    assert got.tolist() == ref.tolist()


def test_int8_checkpoint_fp16_logits(cuda, ckpt):
    sq, sd, prompts = ckpt
    print("case: SmoothQuant checkpoint fp16", flush=True)
    got, lg = _product(sq, prompts, 6, torch.float16, cuda, True)
    ref, lr = _oracle(sd, prompts, 6, torch.float16)
    # logits compared while the two greedy paths agree (a flip changes the next inputs)
    for b in range(len(prompts)):
        for s in range(6):
            err = float((lg[b, s].double() - lr[b, s].double()).abs().max())
            assert err <= 4e-2, f"prompt {b} step {s}: {err}"
            if got[b, s] != ref[b, s]:
                break
