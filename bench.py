"""Benchmark of the Qwen2 token loop on one MI355X.

Headline (BASELINE.json metric): steady decode throughput of the
Qwen2.5-3B-shape model (random-init bf16 weights, tied embeddings) at batch
40 and context 600. One "step" is one greedy decode forward of the 40
sequences (HIP-graph replay): a fresh batch of 600-token prompts is
prefilled, W untimed decode steps follow, then exactly K decode steps are
timed between device synchronisations; value = K * 40 / wall seconds.

Also reported on the same JSON line:
  reference_formula  the reference harness's own figure
                     (test/generate_token.py:58-67): 600 new tokens for
                     the batch, the prefill forward inside the window,
                     600 * 40 / wall -- comparable with the published
                     864.21 tok/s (README.md:99-100);
  prefill_tok_s      the NoPad prefill of the 40 x 600 prompt tokens;
  roofline           paged decode attention at the BASELINE config-2 shape
                     (40 seqs x 600 ctx, H 12 / KVH 2, D 128, bf16, random
                     slot permutation), cycling 28 independent pools
                     (688 MB > the 256 MB MALL), HIP events on the stream
                     that replays the launches;
  decode_step        bytes and time of the steady decode step;
  prefill_attention  the causal prefill attention of the 40 x 600 prompts
                     (3B and 1.5B head shapes), events around 20 launches,
                     causal TFLOP/s (bench.py --prefill-attention alone);
  cpu_baseline       the CPU oracle (oracle/qwen2.py) timed on the host
                     cores for a bounded number of full decode steps.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3|5]
  --config 3 and --config 5 print the line of that BASELINE config instead
  (Qwen2-1.5B through the scheduler; 3B W8A8 with the radix cache).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
B, PROMPT = 40, 600
# HBM bytes per config-2 attention op (one kernel, split merge included), from
# rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of `bench.py --attention-only`,
# scaled by what the counters read for a 256 MiB copy (fetch x2.0, write x1.0).
# Measured on the current kernels; re-measure when they change.
ATTN_TRAFFIC_BYTES = 25676232


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------ attention
def _config2_inputs(dev, pools, L, identity=False):
    H, KVH, D = 12, 2, 128
    P = B * L
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, H, D, generator=g, device=dev).bfloat16()
    pool_list = [torch.randn(P, 2 * KVH, D, generator=g, device=dev).bfloat16() for _ in range(pools)]
    order = np.arange(P) if identity else np.random.RandomState(0).permutation(P)
    perm = torch.from_numpy(order.astype(np.int32)).view(B, L).to(dev)
    rids = torch.arange(B, dtype=torch.int32, device=dev)
    lens = torch.full((B,), L, dtype=torch.int64, device=dev)
    return q, pool_list, perm, rids, lens


def _graph_time(dev, launch, iters, reps=5):
    """Average seconds per launch of `iters` back-to-back launches replayed
    from one HIP graph (events recorded on the replaying stream). The
    launches are warmed up on the stream they are captured on, so the
    library's per-stream workspaces are sized before the capture."""
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(cap):
        for i in range(min(iters, 32)):
            launch(i)  # first use outside the capture (sizes workspaces)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        for i in range(iters):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (iters * reps)


def bench_decode_attention(dev, iters=200, pools=28, L=600, identity=False):
    """Config 2 (context L): returns (avg seconds per launch, algorithmic bytes
    per launch). identity: slot table = arange instead of the seeded random
    permutation."""
    from lite_lang_amd import ops
    q, pool_list, perm, rids, lens = _config2_inputs(dev, pools, L, identity)
    KVH = 2
    B_, H, D = q.shape
    out = torch.empty_like(q)

    def launch(i):
        p = pool_list[i % pools]
        ops.decode_attention(q, perm, rids, lens, L, p[:, :KVH], p[:, KVH:], out)

    sec = _graph_time(dev, launch, iters)
    nbytes = B * L * 2 * KVH * D * 2 + 2 * B * H * D * 2 + B * L * 4 + B * 8
    return sec, nbytes


def bench_attention_floor(dev, iters=200, pools=28, L=600):
    """What one launch of the config-2 K/V bytes costs at all on this GPU:
    the decode attention itself, a plain contiguous read of each pool (the
    same 24,576,000 K/V bytes) at several grid sizes, and the attention's
    own gather (lengths and rows, slot ids, then every K/V row through the
    slot table, on its split grid, no arithmetic) into registers and into
    LDS. Every figure is one launch per pool, 28 pools cycled (688 MB, past
    the 256 MB MALL), timed as the attention is (graph replay, events)."""
    from lite_lang_amd import _lib, ops
    Lb = _lib.load()
    q, pool_list, perm, rids, lens = _config2_inputs(dev, pools, L)
    KVH, D = 2, 128
    out = torch.empty_like(q)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    kv_bytes = B * L * 2 * KVH * D * 2
    assert pool_list[0].numel() * 2 == kv_bytes
    res = {"kv_bytes": kv_bytes, "pools": pools, "launches_per_graph": iters}

    def attn(i):
        p = pool_list[i % pools]
        ops.decode_attention(q, perm, rids, lens, L, p[:, :KVH], p[:, KVH:], out)

    res["attention_us"] = round(_graph_time(dev, attn, iters) * 1e6, 3)
    stream = lambda: torch.cuda.current_stream(dev).cuda_stream
    reads = {}
    for wgs in (256, 512, 1024, 2048, 4096):
        def read(i, wgs=wgs):
            _lib.check(Lb.ll_probe_stream_read(pool_list[i % pools].data_ptr(), kv_bytes, wgs,
                                               sink.data_ptr(), stream()), "ll_probe_stream_read")
        reads[str(wgs)] = round(_graph_time(dev, read, iters) * 1e6, 3)
    res["plain_read_us"] = reads
    ns = int(Lb.ll_decode_attention_split_count(B, KVH, D, L))
    res["split_count"] = ns
    for mode, name in ((0, "gather_registers_us"), (1, "gather_lds_us")):
        def gather(i, mode=mode):
            p = pool_list[i % pools]
            k, v = p[:, :KVH], p[:, KVH:]
            _lib.check(Lb.ll_probe_kv_gather(k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(),
                                              v.stride(0), v.stride(1), perm.data_ptr(),
                                              perm.stride(0), rids.data_ptr(), 0, lens.data_ptr(),
                                              1, B, KVH, D, 2, L, ns, mode, sink.data_ptr(),
                                              stream()), "ll_probe_kv_gather")
        res[name] = round(_graph_time(dev, gather, iters) * 1e6, 3)
    best_read = min(reads.values())
    res["plain_read_best_gbs"] = round(kv_bytes / best_read / 1e3, 1)
    res["gather_best_us"] = min(res["gather_registers_us"], res["gather_lds_us"])
    res["gather_frac_of_peak"] = round(kv_bytes / res["gather_best_us"] / 1e3 / HBM_PEAK_GBS, 4)
    res["plain_read_frac_of_peak"] = round(kv_bytes / best_read / 1e3 / HBM_PEAK_GBS, 4)
    return res


def bench_launch_floor(dev, iters=100):
    """What a launch costs by itself inside a HIP graph (the decode step is
    221 of them): back-to-back launches of an empty 512-thread kernel at
    several grid sizes, and of the same kernel writing 64 KB .. 16 MB with
    16-byte stores (240 workgroups, the decode attention's grid), timed as
    the attention is (graph replay, events). The buffer a launch writes is
    its own (the writes are cold in the L2)."""
    from lite_lang_amd import _lib
    Lb = _lib.load()
    stream = lambda: torch.cuda.current_stream(dev).cuda_stream
    buf = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
    res = {"launches_per_graph": iters, "threads_per_workgroup": 512}
    empty = {}
    for wgs in (1, 240, 256, 1024):
        def launch(i, wgs=wgs):
            _lib.check(Lb.ll_probe_launch(None, 0, wgs, stream()), "ll_probe_launch")
        empty[str(wgs)] = round(_graph_time(dev, launch, iters) * 1e6, 3)
    res["empty_us"] = empty
    writes = {}
    for kb in (64, 256, 1024, 4096, 16384):
        def launch(i, kb=kb):
            off = (i % 2) * (32 << 20)
            _lib.check(Lb.ll_probe_launch(buf.data_ptr() + off, kb * 1024, 240, stream()),
                       "ll_probe_launch")
        writes[str(kb)] = round(_graph_time(dev, launch, iters) * 1e6, 3)
    res["write_kb_us"] = writes
    return res


# ------------------------------------------------------------------ model
def build_runner(dev, cfg, max_length, seed=0):
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    kv_slots = B * max_length * 2 + 1024
    runner = Qwen2ModelRunner(cfg.layer_nums, B, cfg, tp_rank=0, world_size=1, model_path=None,
                              max_length=max_length, mem_usage=0.5, use_radix_cache=False,
                              dtype=torch.bfloat16, seed=seed, kv_max_size=kv_slots, device=dev)
    runner.init_model()
    return runner


def messages(prompt_len, seed):
    rs = np.random.RandomState(seed)
    return [{"id": i, "input_tokens": rs.randint(0, 151936, size=prompt_len).tolist(),
             "temperature": 0.0, "top_p": 1.0, "top_k": 1, "do_sample": False,
             "ignore_eos": True} for i in range(B)]


def steady_decode(runner, msgs, warmup, steps, dev):
    """Prefill a fresh batch (untimed), `warmup` decode steps, then `steps`
    timed decode steps; returns (seconds for the timed steps, prefill seconds)."""
    from lite_lang_amd.models.runner_batch import RunnerBatch
    batch = RunnerBatch.create_batch(msgs, "steady", is_prefill=True, model_runner=runner)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    batch.update_forward_message(runner.forward(batch))
    torch.cuda.synchronize(dev)
    t_prefill = time.perf_counter() - t0
    for _ in range(warmup):
        batch.update_forward_message(runner.forward(batch))
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        batch.update_forward_message(runner.forward(batch))
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    runner.free_reqs(list(batch.request_mapping.values()))
    return wall, t_prefill


def run_window(runner, msgs, n_forwards, dev):
    """The generate_token.py loop: n forwards (prefill first), greedy."""
    from lite_lang_amd.models.runner_batch import RunnerBatch
    batch = RunnerBatch.create_batch(msgs, "bench", is_prefill=True, model_runner=runner)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    t_prefill = None
    for i in range(n_forwards):
        out = runner.forward(batch)
        batch.update_forward_message(out)
        if i == 0:
            torch.cuda.synchronize(dev)
            t_prefill = time.perf_counter() - t0
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    runner.free_reqs(list(batch.request_mapping.values()))
    return wall, t_prefill


# ------------------------------------------------------------------ CPU baseline
def cpu_baseline(seconds=20.0, min_steps=2, max_steps=6):
    """CPU oracle (oracle/qwen2.py) decode steps of the full Qwen2.5-3B shape
    at batch 40, context 600, in float32 arithmetic with bf16 storage
    emulation (the rounding points of the GPU path).

    Sample: all 36 layers and the full lm_head per step; the 36 layers share
    one random layer's weights, which gives each step the same arithmetic and
    the same weight traffic as 36 distinct layers (each layer's 308 MB of
    fp32 weights is far larger than the host caches) without generating 12 GB
    of random weights. The KV pool holds 600 random tokens per request (no
    prefill). One untimed warm-up step, then timed steps until `seconds` or
    max_steps (at least min_steps); the median step gives tok/s = 40 / step.
    """
    from oracle import ops as O
    from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle
    from oracle.runner_batch import Req
    from lite_lang_amd.models.qwen2.weights import Qwen2Config, random_state_dict
    cores = min(os.cpu_count() or 1, 16)  # the GPU box's CPU share
    torch.set_num_threads(cores)
    L = 36
    cfg1 = Qwen2Config(layer_nums=1, hidden_size=2048, num_heads=16, num_key_value_heads=2,
                       intermediate_size=11008, vocab_size=151936)
    sd = random_state_dict(cfg1, seed=0)
    slots = B * (PROMPT + max_steps + 4)
    with O.math_dtype(torch.float32):
        oc = Qwen2Cfg(num_layers=1, hidden=2048, heads=16, kv_heads=2, intermediate=11008,
                      vocab=151936)
        orc = Qwen2Oracle(oc, sd, torch.bfloat16, B, PROMPT + max_steps + 4, slots)
        del sd
        orc.layers = [orc.layers[0]] * L
        orc.cfg.num_layers = L
        g = torch.Generator().manual_seed(1)
        orc.pool = torch.randn((L, slots, 4, 128), generator=g).bfloat16().float()
        reqs = []
        for _ in range(B):
            r = Req(rid=orc.cache.alloc_req(), input_tokens=[0] * PROMPT, output_tokens=[1])
            orc.cache.alloc_token_idxs([r.rid], [0], [PROMPT])
            reqs.append(r)
        ids = [1] * B
        orc.forward(reqs, False, ids)  # warm-up
        for r in reqs:
            r.output_tokens.append(1)
        ts = []
        while len(ts) < max_steps and (len(ts) < min_steps or sum(ts) < seconds):
            t0 = time.perf_counter()
            orc.forward(reqs, False, ids)
            ts.append(time.perf_counter() - t0)
            for r in reqs:
                r.output_tokens.append(1)
    step = float(np.median(ts))
    return {"value": round(B / step, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": (f"CPU oracle (float32 math, bf16 storage emulation), {len(ts)} full "
                       f"decode steps of the Qwen2.5-3B shape (36 layers sharing one random "
                       f"layer's weights, full lm_head) at batch {B}, context {PROMPT}, random "
                       f"KV pool, no prefill; median {step:.3f} s/step after one warm-up "
                       f"(steps {', '.join(f'{t:.3f}' for t in ts)} s)")}


# ------------------------------------------------------------------ configs 3 and 5
def bench_config3(dev, new_tokens=600):
    """Qwen2-1.5B shape, 40 requests x 600 random prompt ids, 600 greedy new
    tokens each, driven end to end by the continuous-batching scheduler
    (admission, prefill, decode bursts of 10, filtering), one token readback
    per step as the reference's scheduler loop does."""
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import qwen2_1p5b_config
    from lite_lang_amd.scheduler import IdTokenizer, LocalModelClient, Scheduler
    cfg = qwen2_1p5b_config()
    max_length = PROMPT + new_tokens + 2
    runner = Qwen2ModelRunner(cfg.layer_nums, B, cfg, max_length=max_length, dtype=torch.bfloat16,
                              seed=0, kv_max_size=B * max_length + 64, device=dev)
    sch = Scheduler(max_batch_size=B, tokenizer=IdTokenizer(eos_token_id=-1),
                    max_total_length=PROMPT + new_tokens, max_output_length=new_tokens,
                    max_reqs=4 * B, model_client=LocalModelClient(runner), busy_scale=0.9)
    # warm-up: one short request through the same path (graph capture of B=1 and kernels),
    # then a prefill + decode step of the benchmark's shape on the runner itself (the
    # vendor GEMMs' first use at M = 24,000 and the batch-40 decode graph capture)
    w = sch.add_req_tokens(messages(8, seed=9)[0]["input_tokens"])
    while not w.is_end:
        sch.forward()
    run_window(runner, messages(PROMPT, seed=1), 2, dev)
    torch.cuda.synchronize(dev)
    reqs = [sch.add_req_tokens(m["input_tokens"]) for m in messages(PROMPT, seed=3)]
    t0 = time.perf_counter()
    t_prefill = None
    while not all(r.is_end for r in reqs):
        sch.forward()
        if t_prefill is None:
            t_prefill = time.perf_counter() - t0  # first round: prefill + 10 decode steps
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    gen = sum(r.output_length for r in reqs)
    return {"metric": "config 3: generated tok/s Qwen2-1.5B bs40 ctx600 +600 (scheduler, end to end)",
            "value": round(gen / wall, 2), "unit": "tok/s", "n_gpus": 1, "higher_is_better": True,
            "dtype": "bf16", "data": "synthetic (random-init weights, uniform random prompt ids)",
            "config": {"workload": "Qwen2-1.5B shape, 40 x 600-token prompts, 600 greedy tokens each, "
                                   "continuous batching through lite_lang_amd.scheduler",
                       "global_batch": B, "seq_len": PROMPT, "new_tokens": new_tokens},
            "wall_s": round(wall, 3), "generated_tokens": gen,
            "first_round_s": round(t_prefill, 4)}


def bench_config5(dev, steps=300, warmup=2):
    """Qwen2.5-3B shape with W8A8 projections (int8 per-channel weights,
    per-token int8 activations, bf16 lm_head) and the radix cache: a warm
    request leaves a 400-token prefix in the tree; then 40 requests, 32 of
    them starting with that prefix (200 new prompt tokens each) and 8 with
    600 unique tokens, are prefilled and decoded; decode tok/s at batch 40."""
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import qwen25_3b_config
    from lite_lang_amd.models.runner_batch import RunnerBatch
    cfg = qwen25_3b_config()
    max_length = PROMPT + steps + warmup + 8
    runner = Qwen2ModelRunner(cfg.layer_nums, B + 1, cfg, max_length=max_length,
                              dtype=torch.bfloat16, seed=0, kv_max_size=(B + 2) * max_length * 2,
                              device=dev, quant="w8a8", use_radix_cache=True)
    runner.init_model()
    rs = np.random.RandomState(5)
    prefix = rs.randint(0, 151936, size=400).tolist()
    warm = RunnerBatch.create_batch([{"id": 999, "input_tokens": prefix + rs.randint(0, 151936, size=8).tolist()}],
                                    "warm", True, runner)
    for _ in range(3):
        warm.update_forward_message(runner.forward(warm))
    warm.filter([999])
    msgs = []
    for i in range(B):
        toks = (prefix + rs.randint(0, 151936, size=200).tolist()) if i < 32 else \
            rs.randint(0, 151936, size=PROMPT).tolist()
        msgs.append({"id": i, "input_tokens": toks})
    batch = RunnerBatch.create_batch(msgs, "c5", True, runner)
    shared = sum(len(r.shared_tokens) for r in batch.request_mapping.values())
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    batch.update_forward_message(runner.forward(batch))
    torch.cuda.synchronize(dev)
    t_prefill = time.perf_counter() - t0
    for _ in range(warmup):
        batch.update_forward_message(runner.forward(batch))
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        batch.update_forward_message(runner.forward(batch))
    torch.cuda.synchronize(dev)
    dt = time.perf_counter() - t0
    wbytes = runner.model_ins_.w.nbytes_streamed_per_decode()
    # KV rows read per step at the mean context of the timed steps (600-token prompts)
    ctx_mean = PROMPT + 1 + warmup + steps / 2
    kv_bytes = cfg.layer_nums * B * ctx_mean * 2 * cfg.num_key_value_heads * cfg.head_dim * 2
    step_sec = dt / steps
    return {"metric": "config 5: decode tok/s Qwen2.5-3B W8A8 + radix bs40 ctx600",
            "value": round(steps * B / dt, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": round(step_sec * 1e3, 4), "higher_is_better": True,
            "decode_step": {"bytes": int(wbytes + kv_bytes), "weight_bytes": int(wbytes),
                            "kv_bytes": int(kv_bytes),
                            "hbm_frac": round((wbytes + kv_bytes) / step_sec / 1e9 / HBM_PEAK_GBS, 4)},
            "dtype": "int8 x int8 -> int32 (projections), bf16 elsewhere",
            "data": "synthetic (random-init weights quantised per channel, random prompt ids)",
            "config": {"workload": "Qwen2.5-3B shape W8A8, radix on: 32 of 40 prompts share a "
                                   "400-token cached prefix", "global_batch": B, "seq_len": PROMPT},
            "prefill_s": round(t_prefill, 4), "prefix_tokens_reused": shared}


def bench_prefill_attention(dev, reps=20):
    """The causal prefill attention of 40 x 600-token prompts (the 3B shape,
    16 query / 2 KV heads, and the 1.5B shape, 12 / 2; head_dim 128, bf16)
    over a seeded random slot permutation, events around `reps` launches.
    Causal flops: 4 * head_dim * (keys seen, summed over query rows) per
    query head."""
    from lite_lang_amd import ops
    L, D = PROMPT, 128
    T = B * L
    out = {"workload": f"prefill attention {B} x {L}, head_dim {D}, bf16, random slot table"}
    for H, KVH in ((16, 2), (12, 2)):
        g = torch.Generator(device=dev).manual_seed(7)
        q = torch.randn(T, H, D, generator=g, device=dev).bfloat16()
        pool = torch.randn(T + 64, 2 * KVH, D, generator=g, device=dev).bfloat16()
        o = torch.empty_like(q)
        r2t = torch.from_numpy(np.random.RandomState(7).permutation(T).astype(np.int32)).view(B, L).to(dev)
        rids = torch.arange(B, dtype=torch.int32, device=dev)
        start = torch.arange(B, dtype=torch.int32, device=dev) * L
        lens = torch.full((B,), L, dtype=torch.int32, device=dev)

        def run():
            ops.prefill_attention(q, pool[:, :KVH], pool[:, KVH:], o, rids, start, lens, L, r2t)

        run()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize(dev)
        us = e0.elapsed_time(e1) / reps * 1e3
        flops = 4.0 * D * H * B * (L * (L + 1) / 2)
        out[f"h{H}_kv{KVH}"] = {"us": round(us, 1), "tflops": round(flops / us / 1e6, 1),
                                "frac_of_bf16_peak": round(flops / us / 1e6 / 2500.0, 3)}
    return out


def bench_prefill_gemms(dev, M=B * PROMPT, reps=20):
    """The prefill projections of the 3B shape at M = 40 x 600 tokens on the
    tile GEMMs (bf16: qkv, o, gate/up with the SiLU_and_Mul epilogue, down;
    W8A8: the dequantising int8 kernels), events around `reps` launches each."""
    from lite_lang_amd import ops
    from lite_lang_amd.models.qwen2.weights import qwen25_3b_config
    cfg = qwen25_3b_config()
    hd, I = cfg.hidden_size, cfg.intermediate_size
    qkv_n = (cfg.num_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim
    g = torch.Generator(device=dev).manual_seed(5)
    out = {}

    def timed(name, flops, fn):
        fn()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize(dev)
        us = e0.elapsed_time(e1) / reps * 1e3
        out[name] = {"us": round(us, 1), "tflops": round(flops / us / 1e6, 1)}

    for name, N, K in [("qkv", qkv_n, hd), ("o", hd, cfg.num_heads * cfg.head_dim),
                       ("gate_up_silu", 2 * I, hd), ("down", hd, I)]:
        x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        w = (torch.randn(N, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        if name == "gate_up_silu":
            wil = ops.interleave_gate_up(w)
            timed("bf16_" + name, 2.0 * M * N * K, lambda: ops.gate_up_silu_tiled(x, wil))
        else:
            timed("bf16_" + name, 2.0 * M * N * K, lambda: ops.gemm_tiled(x, w))
        qw = ops.QuantWeight(w, gate_up=(name == "gate_up_silu"))
        xq, st = ops.quant_per_token(x)
        if name == "gate_up_silu":
            timed("w8a8_" + name, 2.0 * M * N * K,
                  lambda: ops.gemm_i8_gate_up_silu_tiled(xq, st, qw.q_il, qw.scale))
        else:
            timed("w8a8_" + name, 2.0 * M * N * K,
                  lambda: ops.gemm_i8_tiled(xq, st, qw.q, qw.scale))
        del x, w, qw, xq, st
        torch.cuda.empty_cache()
    return out


def bench_norm_qkv(dev, reps=400, copies=32):
    """The decode step's add + RMSNorm fused with the next layer's QKV
    projection (ops.add_rmsnorm_qkv_splitk) at the 3B shape, batch 40: the
    down_proj partials of the real split count, `copies` packed QKV weights
    cycled (336 MB, past the 256 MB MALL), events around `reps` launches.
    Algorithmic bytes per launch: down partials read, residual read and
    written, gain, normalised rows written and read once by the QKV items,
    the QKV weight, the QKV partials written."""
    from lite_lang_amd import ops, _lib
    from lite_lang_amd.models.qwen2.weights import qwen25_3b_config
    cfg = qwen25_3b_config()
    hd, I = cfg.hidden_size, cfg.intermediate_size
    nqkv = (cfg.num_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim
    dsplits = int(_lib.load().ll_gemm_splitk_count(B, hd, I))
    qs = ops.add_rmsnorm_qkv_splits(B, hd, nqkv)
    g = torch.Generator(device=dev).manual_seed(7)
    wps = [ops.PackedWeight((torch.randn(nqkv, hd, device=dev, generator=g) * 0.02)
                            .to(torch.bfloat16)) for _ in range(copies)]
    gamma = (torch.rand(hd, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    part = torch.randn(dsplits * B * hd, device=dev, generator=g) * 0.3
    qpart = torch.empty(qs * B * nqkv, device=dev)
    h = torch.randn(B, hd, device=dev, generator=g).to(torch.bfloat16)
    x = torch.empty_like(h)
    ops.decode_sync(dev)
    ops.reserve_workspace(dev, "decode_epoch", 4)

    def call(i):
        ops.add_rmsnorm_qkv_splitk(h, part, dsplits, gamma, cfg.rms_norm_eps, wps[i % copies],
                                   qpart, ops.decode_epoch_advance(dev), tag=i % 200, x=x)

    for i in range(copies):
        call(i)
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        call(i)
    e1.record()
    torch.cuda.synchronize(dev)
    us = e0.elapsed_time(e1) / reps * 1e3  # includes the epoch-advance launch
    nbytes = (dsplits * B * hd * 4 + 2 * B * hd * 2 + hd * 2 + 2 * B * hd * 2
              + nqkv * hd * 2 + qs * B * nqkv * 4)
    assert ops.decode_sync_status(dev) == 0
    return {"kernel": "norm_qkv_kernel (add + RMSNorm + next QKV, Qwen2.5-3B, batch 40)",
            "us_per_call_with_epoch_advance": round(us, 3), "bytes_per_launch": nbytes,
            "down_splits": dsplits, "qkv_splits": qs}


# ------------------------------------------------------------------ main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave configs 3 and 5 out of the default line")
    ap.add_argument("--config", type=int, default=4, choices=(3, 4, 5),
                    help="4: the headline line (default); 3: Qwen2-1.5B through the scheduler; "
                         "5: 3B W8A8 + radix cache")
    ap.add_argument("--attention-sweep", action="store_true",
                    help="time the config-2 decode attention at contexts 16..2400 (random "
                         "slot table; identity table at 600 and 1200), one JSON line each")
    ap.add_argument("--prefill-gemm", action="store_true",
                    help="time the 3B prefill projections (M = 24,000) on the tile GEMMs, "
                         "bf16 and W8A8, one JSON line")
    ap.add_argument("--prefill-attention", action="store_true",
                    help="time the 40 x 600 causal prefill attention (3B and 1.5B head "
                         "shapes), one JSON line")
    ap.add_argument("--attention-only", action="store_true",
                    help="run only the config-2 decode attention launches plus a 256 MiB "
                         "device copy of known size (for rocprofv3 --pmc traffic runs)")
    ap.add_argument("--attention-floor", action="store_true",
                    help="time the config-2 decode attention beside a plain read and a slot-table "
                         "gather of the same K/V bytes (in-tree probe kernels), one JSON line")
    ap.add_argument("--launch-floor", action="store_true",
                    help="time graph-replayed launches of an empty kernel and of kernels that "
                         "write 64 KB .. 16 MB (in-tree probe kernel), one JSON line")
    ap.add_argument("--norm-qkv", action="store_true",
                    help="run only the fused add + RMSNorm + QKV launch of the 3B decode step "
                         "plus a 256 MiB device copy of known size (for rocprofv3 runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU (tp=1, no collectives); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    from lite_lang_amd.models.qwen2.weights import qwen25_3b_config
    cfg = qwen25_3b_config()
    K, W = args.steps, args.warmup

    if args.config == 3:
        print(json.dumps(bench_config3(dev)), flush=True)
        return
    if args.config == 5:
        print(json.dumps(bench_config5(dev)), flush=True)
        return

    if args.attention_sweep:
        for L, ident in [(16, False), (64, False), (150, False), (300, False), (600, False),
                         (1200, False), (2400, False), (600, True), (1200, True)]:
            sec, nb = bench_decode_attention(dev, L=L, identity=ident)
            print(json.dumps({"ctx": L, "slots": "identity" if ident else "random",
                              "us": round(sec * 1e6, 3), "bytes": nb,
                              "gbs": round(nb / sec / 1e9, 1)}), flush=True)
            torch.cuda.empty_cache()
        return
    if args.attention_floor:
        print(json.dumps(bench_attention_floor(dev)), flush=True)
        return
    if args.launch_floor:
        print(json.dumps(bench_launch_floor(dev)), flush=True)
        return
    if args.prefill_gemm:
        print(json.dumps(bench_prefill_gemms(dev)), flush=True)
        return
    if args.prefill_attention:
        print(json.dumps(bench_prefill_attention(dev)), flush=True)
        return
    if args.norm_qkv:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)  # reference copy: 256 MiB read + 256 MiB written
        torch.cuda.synchronize()
        print(json.dumps(bench_norm_qkv(dev)), flush=True)
        return
    if args.attention_only:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)  # reference copy: 256 MiB read + 256 MiB written
        torch.cuda.synchronize()
        attn_sec, attn_bytes = bench_decode_attention(dev, iters=50)
        print(json.dumps({"attention_us": attn_sec * 1e6, "bytes_per_launch": attn_bytes}))
        return

    log("decode attention microbench (config 2)")
    attn_sec, attn_bytes = bench_decode_attention(dev)
    attn_gbs = attn_bytes / attn_sec / 1e9
    log(f"attention: {attn_sec * 1e6:.2f} us, {attn_gbs:.0f} GB/s")
    # the same op at twice the context: the extra bytes over the extra time is
    # the rate the op streams at beyond its fixed per-launch cost
    sec2, bytes2 = bench_decode_attention(dev, L=2 * PROMPT)
    marg_gbs = (bytes2 - attn_bytes) / (sec2 - attn_sec) / 1e9
    fixed_us = (attn_sec - attn_bytes / (marg_gbs * 1e9)) * 1e6
    log(f"attention at ctx {2 * PROMPT}: {sec2 * 1e6:.2f} us; marginal {marg_gbs:.0f} GB/s, "
        f"fixed {fixed_us:.2f} us")

    log("attention floor: plain read and gather of the same K/V bytes")
    floor = bench_attention_floor(dev)
    log(f"floor: plain read {min(floor['plain_read_us'].values()):.2f} us, gather "
        f"{floor['gather_best_us']:.2f} us")
    torch.cuda.empty_cache()

    log("building Qwen2.5-3B-shape runner (random init, bf16)")
    ref_new = PROMPT  # the reference harness generates 600 tokens per request
    max_length = PROMPT + max(ref_new, W + K + 1) + 2
    runner = build_runner(dev, cfg, max_length)
    log("warmup: prefill + 2 decode steps (graph capture, first use of every kernel)")
    run_window(runner, messages(PROMPT, seed=1), 3, dev)
    log(f"steady decode: prefill, {W} untimed steps, {K} timed steps")
    wall, t_prefill = steady_decode(runner, messages(PROMPT, seed=2), W, K, dev)
    value = K * B / wall
    step_sec = wall / K
    wbytes = runner.model_ins_.w.nbytes_streamed_per_decode()
    kv_ctx_mean = PROMPT + 1 + W + K / 2
    step_bytes = wbytes + cfg.layer_nums * B * kv_ctx_mean * 2 * cfg.num_key_value_heads * cfg.head_dim * 2
    log(f"steady decode {step_sec * 1e3:.3f} ms/step = {value:.1f} tok/s; "
        f"prefill {t_prefill * 1e3:.1f} ms")
    log(f"reference-harness window: prefill + {ref_new - 1} decode steps")
    ref_wall, ref_prefill = run_window(runner, messages(PROMPT, seed=3), ref_new, dev)
    ref_value = ref_new * B / ref_wall
    log(f"reference formula {ref_value:.1f} tok/s ({ref_wall:.3f} s window)")

    del runner
    torch.cuda.empty_cache()
    configs = None
    if not args.no_configs:
        configs = {}
        for name, fn in (("config3", bench_config3), ("config5", bench_config5)):
            log(f"{name}")
            try:
                sub = fn(dev)
            except Exception as e:  # reported in the line, the headline still stands
                sub = {"error": repr(e)}
            configs[name] = {k: v for k, v in sub.items() if k not in ("n_gpus", "higher_is_better")}
            log(f"{name}: {sub.get('value')} {sub.get('unit', '')}")
            torch.cuda.empty_cache()
    log("prefill attention")
    try:
        prefill_attn = bench_prefill_attention(dev)
    except Exception as e:  # reported in the line, the headline still stands
        prefill_attn = {"error": repr(e)}
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle)")
        try:
            cpu = cpu_baseline()
        except Exception as e:  # reported, not fatal
            cpu = {"value": None, "unit": "tok/s", "cores": os.cpu_count(), "kind": "port",
                   "sample": f"failed: {e!r}"}

    res = {
        "metric": "decode tok/s Qwen2.5-3B bs40 ctx600 + paged-decode attn % HBM peak",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(step_sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / 864.21, 3),
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0,0.02), uniform random prompt ids)",
        "config": {"workload": "Qwen2.5-3B-shape steady decode, batch 40, 600-token prompts "
                               "(one step = one decode forward of the batch)",
                   "global_batch": B, "seq_len": PROMPT, "parallelism": "tp1"},
        "reference_formula": {"value": round(ref_value, 2), "unit": "tok/s",
                              "window_s": round(ref_wall, 4), "new_tokens": ref_new,
                              "vs_published": round(ref_value / 864.21, 3),
                              "note": "test/generate_token.py:58-67: prefill + 599 decode "
                                      "forwards inside the window"},
        "prefill_tok_s": round(B * PROMPT / ref_prefill, 1),
        "decode_step": {"ms": round(step_sec * 1e3, 4), "bytes": int(step_bytes),
                        "hbm_frac": round(step_bytes / step_sec / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline": {"kernel": "decode_attn_dma_kernel (config 2; split merge in the same launch)",
                     "bound": "hbm",
                     "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn_gbs / HBM_PEAK_GBS, 4), "traffic": ATTN_TRAFFIC_BYTES,
                     "avg_us": round(attn_sec * 1e6, 3), "bytes_per_launch": attn_bytes,
                     "marginal": {"ctx": [PROMPT, 2 * PROMPT],
                                  "us": [round(attn_sec * 1e6, 3), round(sec2 * 1e6, 3)],
                                  "gbs": round(marg_gbs, 1),
                                  "frac": round(marg_gbs / HBM_PEAK_GBS, 4),
                                  "fixed_us": round(fixed_us, 3)},
                     "floor": {"plain_read_us": min(floor["plain_read_us"].values()),
                               "plain_read_frac": floor["plain_read_frac_of_peak"],
                               "gather_us": floor["gather_best_us"],
                               "gather_frac": floor["gather_frac_of_peak"],
                               "note": "one launch over the same 24,576,000 K/V bytes: a "
                                       "contiguous read (best grid), and the op's own gather "
                                       "(same grid and dependent loads, no arithmetic); "
                                       "bench.py --attention-floor"}},
        "configs": configs,
        "prefill_attention": prefill_attn,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
