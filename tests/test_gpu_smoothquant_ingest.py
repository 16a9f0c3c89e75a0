"""SmoothQuant checkpoint ingestion on the GPU: the converter's output
(tests/hf_tiny.py:make_smoothquant_checkpoint; int8 weights, fp16
weight_scale, static quant_scale on o_proj/down_proj, pytorch_model.bin)
loaded through model_path -- the runner detects the int8 checkpoint and runs
its W8A8 runtime -- against the CPU oracle reading the same files.

fp32 storage gives the oracle's greedy tokens exactly (the int32 products
are exact and the dequantisation is evaluated in the same fp32 order); fp16
storage, the checkpoint's own dtype, is compared teacher-forced on the logits
of a prefill and decode steps (see that test for the bars: an activation
rounding can flip an int8 code). Both the static quantiser (quant_scale) and
the per-token one run in every layer.
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
    """fp16 storage. The oracle is teacher-forced with the product's tokens,
    so both evaluate every step on the same context. The static and per-token
    quantisers are step functions of their fp16 inputs: a one-ulp difference
    in an activation (another summation order in any kernel) can move an int8
    code by one step, and in this 256-wide model one such flip in the first
    layer's attention output moved a prompt's logits by 0.67 (two prefill
    attention kernels, both within 0.0016 of the oracle's attention, one
    flipping and one not). So: every (prompt, step) within 1.0 (a broken
    kernel moves logits by whole units), the median within 4e-2, and the
    product's token equal to the oracle's argmax wherever the oracle's top-1
    margin exceeds 4x the logits difference of that step."""
    from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle
    sq, sd, prompts = ckpt
    print("case: SmoothQuant checkpoint fp16", flush=True)
    n_new = 6
    got, lg = _product(sq, prompts, n_new, torch.float16, cuda, True)
    oc = Qwen2Cfg(num_layers=2, hidden=256, heads=4, kv_heads=2, intermediate=688, vocab=1024)
    ref, lr = Qwen2Oracle(oc, sd, torch.float16, 8, 128, 1024, quant="w8a8").generate(
        prompts, n_new, return_logits=True, feed=got)
    errs = []
    for b in range(len(prompts)):
        for s in range(n_new):
            err = float((lg[b, s].double() - lr[b, s].double()).abs().max())
            errs.append(err)
            assert err <= 1.0, f"prompt {b} step {s}: {err}"
            top2 = lr[b, s].double().topk(2).values
            if float(top2[0] - top2[1]) > 4 * err:
                assert int(got[b, s]) == int(ref[b, s]), f"prompt {b} step {s}: token differs"
    errs.sort()
    assert errs[len(errs) // 2] <= 4e-2, f"median logits difference {errs[len(errs) // 2]}"
    print(f"fp16 W8A8: logits diff median {errs[len(errs) // 2]:.4f}, max {errs[-1]:.4f}", flush=True)
