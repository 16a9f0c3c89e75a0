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

from oracle import ops as O
from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle

pytestmark = pytest.mark.gpu


def _cfgs():
    from lite_lang_amd.models.qwen2.weights import tiny_config
    c = tiny_config()
    oc = Qwen2Cfg(num_layers=c.layer_nums, hidden=c.hidden_size, heads=c.num_heads,
                  kv_heads=c.num_key_value_heads, intermediate=c.intermediate_size,
                  vocab=c.vocab_size, tie_word_embeddings=c.tie_word_embeddings)
    return c, oc


def _run_product(cfg, sd, prompts, n_new, dtype, cuda, max_length=128, graph=True):
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.runner_batch import RunnerBatch
    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, tp_rank=0, world_size=1, model_path=None,
                              max_length=max_length, mem_usage=0.5, use_radix_cache=False,
                              dtype=dtype, state_dict=sd, kv_max_size=1024, device=cuda,
                              use_cuda_graph=graph)
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


@pytest.mark.parametrize("graph", [True, False])
def test_config1_fp32_greedy_tokens_identical(cuda, graph):
    from lite_lang_amd.models.qwen2.weights import random_state_dict
    cfg, ocfg = _cfgs()
    sd = random_state_dict(cfg, seed=0)
    prompt = torch.randint(0, 1024, (16,), generator=torch.Generator().manual_seed(0)).tolist()
    print(f"case: config1 fp32 greedy 32 graph={graph}", flush=True)
    ref = Qwen2Oracle(ocfg, sd, torch.float32, 8, 128, 1024).generate([prompt], 32)
    got, _ = _run_product(cfg, sd, [prompt], 32, torch.float32, cuda, graph=graph)
    assert got.tolist() == ref.tolist()


def test_token_ring_wraps(cuda):
    """150 decode steps: the host token ring (64 rows) wraps twice, retiring its
    oldest row each step; every request's output_tokens must equal the tokens
    the device produced, in order."""
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import random_state_dict
    from lite_lang_amd.models.runner_batch import RunnerBatch
    cfg, _ = _cfgs()
    sd = random_state_dict(cfg, seed=3)
    print("case: token ring 150 steps batch 3", flush=True)
    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, tp_rank=0, world_size=1, model_path=None,
                              max_length=256, mem_usage=0.5, use_radix_cache=False,
                              dtype=torch.bfloat16, state_dict=sd, kv_max_size=2048, device=cuda,
                              use_cuda_graph=True)
    runner.init_model()
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in (5, 12, 9)]
    msgs = [{"id": i, "input_tokens": p, "temperature": 0.0, "top_p": 1.0, "top_k": 1,
             "do_sample": False} for i, p in enumerate(prompts)]
    batch = RunnerBatch.create_batch(msgs, "ring", is_prefill=True, model_runner=runner)
    seen = []
    for _ in range(150):
        out = runner.forward(batch)
        seen.append(out.view(-1).cpu().clone())
        batch.update_forward_message(out)
    want = torch.stack(seen, 1).tolist()
    got = [r.output_tokens for r in batch.request_mapping.values()]
    assert got == want


@pytest.mark.parametrize("graph", [True, False])
def test_tiny_bf16_ragged_batch_logits(cuda, graph):
    from lite_lang_amd.models.qwen2.weights import random_state_dict
    cfg, ocfg = _cfgs()
    sd = random_state_dict(cfg, seed=1)
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in (16, 5, 40)]
    print("case: tiny bf16 ragged batch", flush=True)
    ref, ref_logits = Qwen2Oracle(ocfg, sd, torch.bfloat16, 8, 128, 1024).generate(
        prompts, 8, return_logits=True)
    got, got_logits = _run_product(cfg, sd, prompts, 8, torch.bfloat16, cuda, graph=graph)
    for b in range(len(prompts)):
        for s in range(8):
            d = float((got_logits[b, s].double() - ref_logits[b, s]).abs().max())
            assert d <= 2e-2, f"request {b} step {s}: logits max-abs {d}"
            if got[b, s] != ref[b, s]:
                top2 = ref_logits[b, s].topk(2).values
                assert float(top2[0] - top2[1]) <= 2e-2, "token divergence without a near tie"
                break


@pytest.mark.parametrize("graph", [True, False])
def test_fp32_free_running_32_steps_moving_tokens(cuda, graph):
    """Config-1 geometry in fp32 on weights whose greedy tokens move
    (tests/model_weights.moving_state_dict, seed 44): 1 prefill + 31 decode
    forwards run free (each step feeds its own token), and all 32 tokens
    equal the oracle's. The oracle's sequence is asserted to move and to have
    no near tie (every top-1 margin above 1e-3, far above fp32 rounding), so
    the identity says something about every step's KV reads."""
    from tests.model_weights import moving_state_dict
    cfg, ocfg = _cfgs()
    sd = moving_state_dict(cfg, seed=44)
    prompt = torch.randint(0, 1024, (16,), generator=torch.Generator().manual_seed(44)).tolist()
    print(f"case: fp32 free-running 32 steps, moving weights, graph={graph}", flush=True)
    ref, ref_logits = Qwen2Oracle(ocfg, sd, torch.float32, 8, 128, 1024).generate(
        [prompt], 32, return_logits=True)
    top2 = ref_logits[0].double().topk(2, dim=-1).values
    assert float((top2[:, 0] - top2[:, 1]).min()) > 1e-3
    assert len(set(ref[0].tolist())) >= 8, f"oracle tokens barely move: {ref[0].tolist()}"
    got, _ = _run_product(cfg, sd, [prompt], 32, torch.float32, cuda, graph=graph)
    assert got.tolist() == ref.tolist()


def test_post_layer_logits_within_2e2_of_fp32(cuda):
    """The post layer (post_layer.py:14-24,43-45,75-77) as the decode step
    runs it, at the Qwen2.5-3B shape: final RMSNorm (eps 1e-5) of 40 bf16
    hidden rows, the tied lm_head [151936, 2048] streamed from the packed
    weight with fp32 output, first-index argmax. Against the fp32 reference
    of the same op on the same bf16 inputs (float64 arithmetic): logits
    within max-abs 2e-2 (observed ~1e-5 with the normalised rows rounded to
    bf16 as the reference stores them, a few 1e-3 without that rounding);
    the token equals the reference's wherever the top-1 margin exceeds twice
    the logits difference (most rows here)."""
    from lite_lang_amd import ops
    g = torch.Generator().manual_seed(45)
    h = (torch.randn(40, 2048, generator=g) * 2.0).bfloat16()
    gamma = (torch.rand(2048, generator=g) * 0.4 + 0.8).bfloat16()
    emb = (torch.randn(151936, 2048, generator=g) * 0.02).bfloat16()
    print("case: post layer logits fp32 at the 3B shape", flush=True)
    hd, gd = h.to(cuda), gamma.to(cuda)
    wp = ops.PackedWeight(emb.to(cuda))
    y = ops.rmsnorm(hd, gd, 1e-5)
    logits = ops.gemm_packed(y, wp, out_dtype=torch.float32)
    toks = ops.argmax(logits)
    assert logits.dtype == torch.float32
    got = logits.double().cpu()
    yr = O.rmsnorm(h.double(), gamma.double(), 1e-5)
    ref_rounded = yr.bfloat16().double() @ emb.double().t()
    ref_exact = yr @ emb.double().t()
    d1 = float((got - ref_rounded).abs().max())
    d2 = float((got - ref_exact).abs().max())
    print(f"logits max-abs vs fp32 reference: {d1:.2e} (bf16 row), {d2:.2e} (unrounded row)",
          flush=True)
    assert d1 <= 2e-2 and d2 <= 2e-2
    assert d1 <= 1e-3
    top2 = ref_rounded.topk(2, dim=-1)
    decisive = 0
    for b in range(40):
        d = float((got[b] - ref_rounded[b]).abs().max())
        if float(top2.values[b, 0] - top2.values[b, 1]) > 2 * d:
            decisive += 1
            assert int(toks[b]) == int(top2.indices[b, 0]), b
    assert decisive >= 30


def test_qwen25_3b_geometry_two_layers_batch40(cuda):
    """Qwen2.5-3B layer geometry (hidden 2048, 16/2 heads, D 128, I 11008,
    vocab 151936) with 2 layers, batch 40: exercises the wide-N LDS GEMM, the
    split-K fused decode layer and the graph path at the real shapes.

    The logits are O(5). Two bars, both absolute, at every step for the
    requests whose history still equals both oracles':
      * within 0.05 of the oracle that stores the same bf16 intermediates
        the product stores (the algorithm the product runs, in float64
        arithmetic; 0.035 observed). At logits of this size bf16 rounding
        flips alone exceed the north-star 0.02: the same oracle run in fp32
        instead of float64 arithmetic is 0.033 away from itself (median
        0.02). The config tests, whose logits are within 1.7, hold the
        product to 0.02;
      * within 0.1 of the oracle that keeps every intermediate in fp32. A
        bf16 model cannot meet 0.02 there: the bf16-storage oracle, an
        exact execution of the reference algorithm in bf16, is itself
        0.062-0.064 away from it.
    Tokens must match the bf16 oracle except at near ties (a top-1 margin
    within twice the observed logits difference).
    """
    from lite_lang_amd.models.qwen2.weights import Qwen2Config, random_state_dict
    cfg = Qwen2Config(layer_nums=2, hidden_size=2048, num_heads=16, num_key_value_heads=2,
                      intermediate_size=11008, vocab_size=151936)
    ocfg = Qwen2Cfg(num_layers=2, hidden=2048, heads=16, kv_heads=2, intermediate=11008,
                    vocab=151936)
    sd = random_state_dict(cfg, seed=3)
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, 151936, (int(n),), generator=g).tolist()
               for n in torch.randint(1, 24, (40,), generator=g)]
    print("case: 3B geometry 2 layers batch 40", flush=True)
    tb, lb = Qwen2Oracle(ocfg, sd, torch.bfloat16, 48, 64, 2048).generate(
        prompts, 3, return_logits=True)
    tf, lf = Qwen2Oracle(ocfg, sd, torch.float32, 48, 64, 2048).generate(
        prompts, 3, return_logits=True)
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.runner_batch import RunnerBatch
    runner = Qwen2ModelRunner(2, 48, cfg, max_length=64, dtype=torch.bfloat16, state_dict=sd,
                              kv_max_size=2048, device=cuda)
    runner.init_model()
    msgs = [{"id": i, "input_tokens": p} for i, p in enumerate(prompts)]
    batch = RunnerBatch.create_batch(msgs, "b", True, runner)
    alive = torch.ones(40, dtype=torch.bool)  # requests whose history equals both oracles'
    for step in range(3):
        out = runner.forward(batch)
        lg = runner.model_ins_.last_logits.double().cpu()
        got = out.view(-1).cpu()
        batch.update_forward_message(out)
        err_b = float((lg[alive] - lb[alive, step]).abs().max())
        err_f = float((lg[alive] - lf[alive, step]).abs().max())
        err_bf = float((lb[alive, step] - lf[alive, step]).abs().max())
        print(f"step {step}: |gpu - bf16 oracle| {err_b:.4f}  |gpu - fp32 oracle| {err_f:.4f}  "
              f"|bf16 oracle - fp32 oracle| {err_bf:.4f}", flush=True)
        assert err_b <= 0.05, f"step {step}: {err_b} from the bf16-storage oracle"
        assert err_f <= 0.1, f"step {step}: {err_f} from the fp32 oracle"
        mism = (got != tb[:, step]) & alive
        for b in mism.nonzero().view(-1).tolist():
            top2 = lb[b, step].topk(2).values
            d = float((lg[b] - lb[b, step]).abs().max())
            assert float(top2[0] - top2[1]) <= 2 * d, f"request {b} diverged without a near tie"
        alive &= ~mism & (tb[:, step] == tf[:, step])
    assert int(alive.sum()) >= 30


@pytest.mark.parametrize("graph", [True, False])
def test_radix_prefix_reuse_greedy_tokens(cuda, graph):
    """Config-5 flow on the tiny fp32 model: request 0 (prompt P) finishes and
    is inserted into the radix tree (runner_batch.py:184-204); request 1
    (prompt P + 3 tokens) then matches the cached prefix at admission
    (runner_batch.py:118-147), takes its slots without recomputing them, and
    runs the prompt-cache prefill (flash_attn_v2.py:699-762) on the suffix.
    Both requests' greedy tokens must equal the oracle's full recomputation."""
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import random_state_dict
    from lite_lang_amd.models.runner_batch import RunnerBatch
    cfg, ocfg = _cfgs()
    sd = random_state_dict(cfg, seed=2)
    g = torch.Generator().manual_seed(2)
    P = torch.randint(0, 1024, (20,), generator=g).tolist()
    Q = P + torch.randint(0, 1024, (3,), generator=g).tolist()
    print(f"case: radix prefix reuse graph={graph}", flush=True)
    orc = Qwen2Oracle(ocfg, sd, torch.float32, 8, 128, 1024)
    ref0 = orc.generate([P], 4)[0].tolist()
    ref1 = Qwen2Oracle(ocfg, sd, torch.float32, 8, 128, 1024).generate([Q], 6)[0].tolist()

    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, max_length=128, dtype=torch.float32,
                              state_dict=sd, kv_max_size=1024, device=cuda, use_radix_cache=True,
                              use_cuda_graph=graph)
    runner.init_model()
    b0 = RunnerBatch.create_batch([{"id": 0, "input_tokens": P}], "b0", True, runner)
    for _ in range(4):
        b0.update_forward_message(runner.forward(b0))
    assert b0.request_mapping[0].output_tokens == ref0
    slots0 = runner.kv_cache.get_token_index([b0.request_mapping[0]]).tolist()
    b0.filter([0])  # finish: P + 3 generated tokens go into the tree
    assert runner.radix_cache.all_taken_tokens_ == len(P) + 3

    b1 = RunnerBatch.create_batch([{"id": 1, "input_tokens": Q}], "b1", True, runner)
    req = b1.request_mapping[1]
    cached = P + ref0[:3]
    expect_shared = 0
    for a, b in zip(Q[:-1], cached):
        if a != b:
            break
        expect_shared += 1
    assert len(req.shared_tokens) == expect_shared >= len(P)
    assert req.shared_tokens + req.input_tokens == Q
    for _ in range(6):
        b1.update_forward_message(runner.forward(b1))
    assert b1.request_mapping[1].output_tokens == ref1
    # the shared prefix is served from request 0's slots
    slots1 = runner.kv_cache.get_token_index([req]).tolist()
    assert slots1[:expect_shared] == slots0[:expect_shared]


def _w8a8_cfgs():
    from lite_lang_amd.models.qwen2.weights import Qwen2Config
    c = Qwen2Config(layer_nums=2, hidden_size=256, num_heads=4, num_key_value_heads=2,
                    intermediate_size=768, vocab_size=1024)  # every K a multiple of 256
    oc = Qwen2Cfg(num_layers=2, hidden=256, heads=4, kv_heads=2, intermediate=768, vocab=1024)
    return c, oc


@pytest.mark.parametrize("graph", [True, False])
def test_w8a8_bf16_ragged_batch_logits(cuda, graph):
    """W8A8 model (config 5 numerics) against the W8A8 oracle: int8 per-channel
    weights, per-token int8 activations, exact int32 sums, fp32 dequant. The
    90-token prefill runs the M > 64 library int8 GEMM, the decode steps the
    int8 streaming kernel. Logits within 4e-2 up to the first token
    divergence, which must be a near tie of the oracle. The bar is twice the
    bf16 model's: the per-token quantiser is a step function, so a one-ulp
    bf16 difference in its input (fp32 reductions here, fp64 in the oracle)
    can move an int8 code by one step, worth s_t * s_o * |q_w| (about 2e-3
    at these scales) in every output channel it feeds. The fp32 test below
    shows the integer path itself is exact (identical greedy tokens)."""
    from lite_lang_amd.models.qwen2.weights import random_state_dict
    cfg, ocfg = _w8a8_cfgs()
    sd = random_state_dict(cfg, seed=5)
    g = torch.Generator().manual_seed(5)
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in (40, 30, 20)]
    print(f"case: w8a8 bf16 ragged graph={graph}", flush=True)
    ref, ref_logits = Qwen2Oracle(ocfg, sd, torch.bfloat16, 8, 128, 1024, quant="w8a8").generate(
        prompts, 8, return_logits=True)
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.runner_batch import RunnerBatch
    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, max_length=128, dtype=torch.bfloat16,
                              state_dict=sd, kv_max_size=1024, device=cuda, use_cuda_graph=graph,
                              quant="w8a8")
    runner.init_model()
    batch = RunnerBatch.create_batch([{"id": i, "input_tokens": p} for i, p in enumerate(prompts)],
                                     "b", True, runner)
    logits, toks = [], []
    for _ in range(8):
        out = runner.forward(batch)
        logits.append(runner.model_ins_.last_logits.float().cpu())
        toks.append(out.view(-1).cpu())
        batch.update_forward_message(out)
    got, got_logits = torch.stack(toks, 1), torch.stack(logits, 1)
    worst = 0.0
    for b in range(len(prompts)):
        for s in range(8):
            d = float((got_logits[b, s].double() - ref_logits[b, s]).abs().max())
            worst = max(worst, d)
            assert d <= 4e-2, f"request {b} step {s}: logits max-abs {d}"
            if got[b, s] != ref[b, s]:
                top2 = ref_logits[b, s].topk(2).values
                assert float(top2[0] - top2[1]) <= 4e-2, "token divergence without a near tie"
                break
    print(f"w8a8 bf16 logits max-abs vs oracle: {worst:.4f}")


def test_w8a8_fp32_greedy_tokens_identical(cuda):
    from lite_lang_amd.models.qwen2.weights import random_state_dict
    cfg, ocfg = _w8a8_cfgs()
    sd = random_state_dict(cfg, seed=6)
    prompt = torch.randint(0, 1024, (16,), generator=torch.Generator().manual_seed(6)).tolist()
    print("case: w8a8 fp32 greedy", flush=True)
    ref = Qwen2Oracle(ocfg, sd, torch.float32, 8, 128, 1024, quant="w8a8").generate([prompt], 24)
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.runner_batch import RunnerBatch
    runner = Qwen2ModelRunner(cfg.layer_nums, 8, cfg, max_length=128, dtype=torch.float32,
                              state_dict=sd, kv_max_size=1024, device=cuda, quant="w8a8")
    runner.init_model()
    batch = RunnerBatch.create_batch([{"id": 0, "input_tokens": prompt}], "b", True, runner)
    for _ in range(24):
        batch.update_forward_message(runner.forward(batch))
    assert batch.request_mapping[0].output_tokens == ref[0].tolist()
