"""add + RMSNorm fused with the next layer's QKV projection in one launch
(ll_add_rmsnorm_qkv_splitk: norm workgroups flag their rows, the QKV
workgroups hold their weight slices in registers while they wait).

Against the two launches it replaces (ll_add_rmsnorm_splitk and the split-K
GEMM) on the same inputs: residual and normalised rows bit-identical; the QKV
partials, summed over the launch's own k splits, equal the GEMM's sum and a
float32 product of the same rows to float32 rounding. Covered over several
calls on one set of sync words (a new epoch each), with the partials written
over the input partials, inside a HIP graph replayed with eager work in
between, and in the model's decode step (fused against unfused). No flag wait
gave up (ll_decode_sync_status)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ops():
    from lite_lang_amd import ops
    return ops


def _case(g, M, hidden, nqkv, splits, dt, cuda):
    ops = _ops()
    w = (torch.randn(nqkv, hidden, generator=g) * 0.02).to(dt).to(cuda)
    gamma = (torch.rand(hidden, generator=g) + 0.5).to(dt).to(cuda)
    part = (torch.randn(splits, M, hidden, generator=g) * 0.3).to(cuda).reshape(-1)
    h = torch.randn(M, hidden, generator=g).to(dt).to(cuda)
    return w, ops.PackedWeight(w), gamma, part, h


def _qkv_sum(part, splits, M, nqkv):
    return part[: splits * M * nqkv].view(splits, M, nqkv).sum(0)


@pytest.mark.parametrize("M,hidden,nqkv,splits,dt", [
    (40, 2048, 2560, 8, torch.bfloat16),   # Qwen2.5-3B, batch 40
    (64, 2048, 2560, 8, torch.float16),
    (1, 2048, 2560, 3, torch.bfloat16),
    (40, 1536, 2048, 8, torch.bfloat16),   # Qwen2-1.5B
    (17, 896, 1152, 7, torch.bfloat16),    # Qwen2-0.5B, a shorter last split (4 + 3 chunks)
    (33, 4096, 1536, 5, torch.float16),    # two norm passes per thread
    (40, 2048, 2624, 8, torch.bfloat16),   # an odd number of 64-row tiles
])
def test_norm_qkv_against_two_launches(cuda, M, hidden, nqkv, splits, dt):
    print(f"case: norm+qkv M={M} hidden={hidden} nqkv={nqkv} splits={splits} {dt}", flush=True)
    ops = _ops()
    qs = ops.add_rmsnorm_qkv_splits(M, hidden, nqkv)
    assert 1 <= qs <= 8
    g = torch.Generator().manual_seed(M + hidden + splits)
    w, wp, gamma, part, h0 = _case(g, M, hidden, nqkv, splits, dt, cuda)
    ha, hb = h0.clone(), h0.clone()
    n_out = max(qs, 8) * M * nqkv
    for it in range(3):
        epoch = ops.decode_epoch_advance(cuda)
        xa = ops.add_rmsnorm_splitk(ha, part, splits, gamma, 1e-6)
        ga = torch.zeros(ops.gemm_splitk_count(M, nqkv, hidden) * M * nqkv, device=cuda)
        sa = ops.gemm_splitk_packed(xa, wp, ga)
        if it < 2:
            qpart = torch.full((n_out,), float("nan"), device=cuda)
            xb, sb = ops.add_rmsnorm_qkv_splitk(hb, part, splits, gamma, 1e-6, wp, qpart, epoch,
                                                tag=it)
        else:
            # the partials written over the input partials (the decode layer's use)
            qpart = torch.zeros(max(part.numel(), n_out), device=cuda)
            qpart[: part.numel()].copy_(part)
            xb, sb = ops.add_rmsnorm_qkv_splitk(hb, qpart, splits, gamma, 1e-6, wp, qpart, epoch,
                                                tag=it)
        torch.cuda.synchronize()
        assert sb == qs
        assert torch.equal(ha, hb), f"residual differs at call {it}"
        assert torch.equal(xa, xb), f"normalised rows differ at call {it}"
        got = _qkv_sum(qpart, qs, M, nqkv)
        assert torch.isfinite(got).all(), f"unwritten partials at call {it}"
        torch.testing.assert_close(got, _qkv_sum(ga, sa, M, nqkv), rtol=1e-5, atol=1e-5)
        ref = xb.float() @ w.float().t()
        torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)
    assert ops.decode_sync_status(cuda) == 0


def test_norm_qkv_rejects_uncovered_shape(cuda):
    print("case: norm+qkv uncovered shape", flush=True)
    ops = _ops()
    from lite_lang_amd import _lib
    assert ops.add_rmsnorm_qkv_splits(40, 3584, 4608) == 0  # Qwen2-7B: 72 tiles x 7 splits > 216
    g = torch.Generator().manual_seed(3)
    w, wp, gamma, part, h = _case(g, 40, 3584, 4608, 3, torch.bfloat16, cuda)
    qpart = torch.zeros(8 * 40 * 4608, device=cuda)
    with pytest.raises(_lib.LiteLangError):
        ops.add_rmsnorm_qkv_splitk(h, part, 3, gamma, 1e-6, wp, qpart,
                                   ops.decode_epoch_advance(cuda), tag=0)


def test_norm_qkv_graph_replays(cuda):
    print("case: norm+qkv graph replays", flush=True)
    ops = _ops()
    M, hidden, nqkv, splits, dt = 40, 2048, 2560, 8, torch.bfloat16
    qs = ops.add_rmsnorm_qkv_splits(M, hidden, nqkv)
    g = torch.Generator().manual_seed(9)
    w, wp, gamma, part, h0 = _case(g, M, hidden, nqkv, splits, dt, cuda)
    # eager reference of one replay: two add + norm + QKV steps on one residual
    he = h0.clone()
    q1 = torch.zeros(qs * M * nqkv, device=cuda)
    q2 = torch.zeros_like(q1)
    x1e, _ = ops.add_rmsnorm_qkv_splitk(he, part, splits, gamma, 1e-6, wp, q1,
                                        ops.decode_epoch_advance(cuda), tag=0)
    x2e, _ = ops.add_rmsnorm_qkv_splitk(he, part, splits, gamma, 1e-6, wp, q2,
                                        ops.decode_epoch_advance(cuda), tag=0)
    torch.cuda.synchronize()
    q1e, q2e, x1e, x2e = q1.clone(), q2.clone(), x1e.clone(), x2e.clone()
    stream = torch.cuda.Stream()
    hg = h0.clone()
    x1 = torch.empty_like(hg)
    x2 = torch.empty_like(hg)
    g1 = torch.zeros_like(q1)
    g2 = torch.zeros_like(q1)
    with torch.cuda.stream(stream):
        ops.decode_sync(cuda)
        ops.reserve_workspace(cuda, "decode_epoch", 4)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            epoch = ops.decode_epoch_advance(cuda)
            ops.add_rmsnorm_qkv_splitk(hg, part, splits, gamma, 1e-6, wp, g1, epoch, tag=0, x=x1)
            # a second call in the same replay (another tag) on the updated residual
            ops.add_rmsnorm_qkv_splitk(hg, part, splits, gamma, 1e-6, wp, g2, epoch, tag=1, x=x2)
    for rep in range(5):
        hg.copy_(h0)
        g1.zero_()
        g2.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(x1, x1e) and torch.equal(x2, x2e), f"rows differ at replay {rep}"
        assert torch.equal(hg, he), f"residual differs at replay {rep}"
        assert torch.equal(g1, q1e), f"first call's partials differ at replay {rep}"
        assert torch.equal(g2, q2e), f"second call's partials differ at replay {rep}"
        # eager work on the default stream in between
        ops.add_rmsnorm_qkv_splitk(h0.clone(), part, splits, gamma, 1e-6, wp,
                                   torch.zeros_like(q1), ops.decode_epoch_advance(cuda), tag=5)
        torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        assert ops.decode_sync_status(cuda) == 0
    assert ops.decode_sync_status(cuda) == 0


def _decode_run(cuda, fused, graph, steps=5):
    """Qwen2.5-3B geometry, 2 layers, batch 40, prompts of 300..600 tokens
    (moving-token weights): prefill + `steps` decode forwards."""
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import Qwen2Config
    from lite_lang_amd.models.runner_batch import RunnerBatch
    from tests.model_weights import moving_state_dict
    cfg = Qwen2Config(layer_nums=2, hidden_size=2048, num_heads=16, num_key_value_heads=2,
                      intermediate_size=11008, vocab_size=151936)
    sd = moving_state_dict(cfg, seed=21)
    g = torch.Generator().manual_seed(21)
    prompts = [torch.randint(0, 151936, (int(n),), generator=g).tolist()
               for n in torch.randint(300, 601, (40,), generator=g)]
    runner = Qwen2ModelRunner(2, 48, cfg, max_length=640, dtype=torch.bfloat16, state_dict=sd,
                              kv_max_size=40 * 640, device=cuda, use_cuda_graph=graph)
    runner.init_model()
    runner.model_ins_.fuse_norm_qkv = fused
    batch = RunnerBatch.create_batch([{"id": i, "input_tokens": p} for i, p in enumerate(prompts)],
                                     "b", True, runner)
    out = []
    for _ in range(steps + 1):
        toks = runner.forward(batch)
        out.append((runner.model_ins_.last_logits.float().cpu(), toks.view(-1).cpu()))
        batch.update_forward_message(toks)
    return out


@pytest.mark.parametrize("graph", [True, False])
def test_model_decode_fused_norm_qkv(cuda, graph):
    """The fused launch changes only the order in which the QKV partials are
    summed: every step's logits stay within bf16 rounding of the unfused
    layer's, and the tokens agree (a step feeds its own tokens forward)."""
    print(f"case: model decode fused norm+qkv graph={graph}", flush=True)
    a = _decode_run(cuda, False, graph)
    b = _decode_run(cuda, True, graph)
    agree = total = 0
    for step, ((la, ta), (lb, tb)) in enumerate(zip(a, b)):
        scale = float(la.abs().max())
        torch.testing.assert_close(lb, la, rtol=0.0, atol=0.02 * scale,
                                   msg=lambda m: f"step {step}: {m}")
        agree += int((ta == tb).sum())
        total += ta.numel()
    assert agree >= 0.95 * total, f"tokens agree on {agree} of {total}"
    # the eager path's sync words are the current stream's; a decode graph's
    # are its capture stream's (workspaces are keyed by stream)
    assert _ops().decode_sync_status(cuda) == 0
    if graph:
        from lite_lang_amd.models.qwen2.decode_graph import _capture_stream
        with torch.cuda.stream(_capture_stream(cuda)):
            assert _ops().decode_sync_status(cuda) == 0
