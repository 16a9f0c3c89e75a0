"""Failure handling of the decode step, forced from the host.

The fused add + RMSNorm + QKV launch waits on flags with a bounded number of
polls, and the fused attention's same-launch split merge waits for the other
splits' partials the same way. A wait that gives up sets the step's error word; the step's argmax
then writes token id -1 for every request (ll_argmax_status), and the host
raises DecodeStepError as soon as it reads such a step's tokens, instead of
handing invalid tokens to the requests. The conditions are forced from the
host, so every kernel exits normally: the error word is set before a step,
or the waits run in the library's test mode (they look for a flag value no
producer writes and give up after a few polls).

Also here: the epoch advance inside the embedding launch, the status form
of the argmax, and the decode attention's split merge in a separate kernel
(the fallback the runner takes when the XCD premise of the same-launch merge
does not hold on a machine) against the same-launch merge, bit for bit.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ops():
    from lite_lang_amd import ops
    return ops


def test_argmax_status(cuda):
    ops = _ops()
    g = torch.Generator(device=cuda).manual_seed(3)
    for M, N in [(40, 151936), (3, 1024), (5, 1000)]:
        print(f"case: argmax status M={M} N={N}", flush=True)
        x = torch.randn(M, N, device=cuda, generator=g).bfloat16()
        want = ops.argmax(x)
        st = torch.zeros(1, dtype=torch.int32, device=cuda)
        assert torch.equal(ops.argmax(x, status=st), want)
        assert torch.equal(want.cpu(), x.float().argmax(1).cpu())
        st.fill_(1)
        got = ops.argmax(x, status=st)
        assert torch.equal(got.cpu(), torch.full((M,), -1, dtype=torch.int64))


def test_embedding_rmsnorm_advances_epoch(cuda):
    ops = _ops()
    g = torch.Generator(device=cuda).manual_seed(4)
    table = torch.randn(1000, 2048, device=cuda, generator=g).bfloat16()
    gamma = (torch.rand(2048, device=cuda, generator=g) + 0.5).bfloat16()
    ids = torch.randint(0, 1000, (40,), device=cuda, generator=g)
    ep = torch.full((1,), 41, dtype=torch.int32, device=cuda)
    print("case: embedding rmsnorm epoch", flush=True)
    h0, x0 = ops.embedding_rmsnorm(table, ids, gamma, 1e-6)
    for k in range(3):
        h1, x1 = ops.embedding_rmsnorm(table, ids, gamma, 1e-6, epoch=ep)
        assert torch.equal(h0, h1) and torch.equal(x0, x1)
        assert int(ep.item()) == 42 + k


def test_embedding_rmsnorm_slot_write(cuda):
    """The decode step's slot-table update folded into its first launch:
    embedding + RMSNorm + epoch with slot_write leaves the table, h and out
    exactly as assign_slots followed by the same launch without it."""
    ops = _ops()
    g = torch.Generator(device=cuda).manual_seed(5)
    table = torch.randn(1000, 2048, device=cuda, generator=g).bfloat16()
    gamma = (torch.rand(2048, device=cuda, generator=g) + 0.5).bfloat16()
    B = 40
    ids = torch.randint(0, 1000, (B,), device=cuda, generator=g)
    r2t0 = torch.randint(0, 1 << 20, (48, 720), device=cuda, generator=g, dtype=torch.int32)
    rows = torch.randperm(48, device=cuda, generator=g)[:B].int()
    cols = torch.randint(0, 720, (B,), device=cuda, generator=g, dtype=torch.int32)
    slots = torch.randint(0, 1 << 20, (B,), device=cuda, generator=g, dtype=torch.int32)
    packed = torch.stack([slots, rows, cols]).contiguous()
    print("case: embedding rmsnorm slot write B=40", flush=True)
    want = r2t0.clone()
    ops.assign_slots(want, packed, B)
    ep0 = torch.full((1,), 7, dtype=torch.int32, device=cuda)
    h0, x0 = ops.embedding_rmsnorm(table, ids, gamma, 1e-6, epoch=ep0)
    got = r2t0.clone()
    ep1 = torch.full((1,), 7, dtype=torch.int32, device=cuda)
    h1, x1 = ops.embedding_rmsnorm(table, ids, gamma, 1e-6, epoch=ep1, slot_write=(got, packed))
    torch.cuda.synchronize()
    assert torch.equal(got, want) and not torch.equal(got, r2t0)
    assert torch.equal(h0, h1) and torch.equal(x0, x1)
    assert int(ep1.item()) == 8


def _runner(cuda, graph):
    from lite_lang_amd.models.qwen2 import Qwen2ModelRunner
    from lite_lang_amd.models.qwen2.weights import Qwen2Config
    from tests.model_weights import moving_state_dict
    cfg = Qwen2Config(layer_nums=2, hidden_size=1024, num_heads=8, num_key_value_heads=2,
                      intermediate_size=2816, vocab_size=4096)
    runner = Qwen2ModelRunner(2, 16, cfg, max_length=160, dtype=torch.bfloat16,
                              state_dict=moving_state_dict(cfg, seed=31), kv_max_size=16 * 160,
                              device=cuda, use_cuda_graph=graph)
    runner.init_model()
    return runner


def _batch(runner, tag):
    from lite_lang_amd.models.runner_batch import RunnerBatch
    g = torch.Generator().manual_seed(31)
    prompts = [torch.randint(0, 4096, (int(n),), generator=g).tolist()
               for n in torch.randint(20, 90, (12,), generator=g)]
    return RunnerBatch.create_batch([{"id": i, "input_tokens": p} for i, p in enumerate(prompts)],
                                    tag, True, runner)


def _steps(runner, batch, n):
    for _ in range(n):
        batch.update_forward_message(runner.forward(batch))


def _error_word_stream(cuda, graph):
    from lite_lang_amd.models.qwen2.decode_graph import _capture_stream
    return _capture_stream(cuda) if graph else torch.cuda.current_stream(cuda)


@pytest.mark.parametrize("graph", [True, False])
def test_runner_raises_on_error_word(cuda, graph):
    """An error word set before a decode step makes that step's tokens -1,
    and reading them raises; after reset_decode_fault the steps are valid
    again."""
    from lite_lang_amd.models.runner_batch import DecodeStepError
    ops = _ops()
    runner = _runner(cuda, graph)
    assert runner.model_ins_.norm_qkv_splits(12) > 0
    batch = _batch(runner, "e")
    print(f"case: error word preset graph={graph}", flush=True)
    _steps(runner, batch, 3)  # prefill + 2 decode steps (captures the graph)
    toks = [r.output_tokens[:] for r in batch.request_mapping.values()]
    assert all(t >= 0 for ts in toks for t in ts)
    with torch.cuda.stream(_error_word_stream(cuda, graph)):
        ops.decode_sync_error(cuda).fill_(1)
    torch.cuda.synchronize()
    _steps(runner, batch, 1)
    with pytest.raises(DecodeStepError):
        batch.flush()
    runner.reset_decode_fault()
    with torch.cuda.stream(_error_word_stream(cuda, graph)):
        assert ops.decode_sync_status(cuda) == 0
    _steps(runner, batch, 2)
    batch.flush()
    last = [r.output_tokens[-2:] for r in batch.request_mapping.values()]
    assert all(t >= 0 for ts in last for t in ts)


@pytest.mark.parametrize("graph", [True, False])
def test_runner_raises_when_waits_give_up(cuda, graph):
    """Every flag wait of the fused launch gives up (test mode of the spin
    limit: the waits look for a value no producer writes, 64 polls): the
    items store nothing, every kernel exits, the error word is set, and the
    runner raises on the step's tokens. With the default restored and the
    word reset, the following steps run normally. A captured graph keeps the
    bound it was captured with, so the graph case captures its decode graph
    under the test mode and recaptures after it."""
    from lite_lang_amd.models.runner_batch import DecodeStepError
    ops = _ops()
    runner = _runner(cuda, graph)
    batch = _batch(runner, "w")
    print(f"case: flag waits give up graph={graph}", flush=True)
    _steps(runner, batch, 1 if graph else 3)
    batch.flush()
    ops.set_decode_spin_limit(-64)
    try:
        _steps(runner, batch, 1)
        torch.cuda.synchronize()
    finally:
        ops.set_decode_spin_limit(0)
    with torch.cuda.stream(_error_word_stream(cuda, graph)):
        assert ops.decode_sync_status(cuda) == 1
    with pytest.raises(DecodeStepError):
        batch.flush()
    runner.reset_decode_fault()
    runner._graphs.clear()  # recapture with the default bound
    _steps(runner, batch, 2)
    batch.flush()
    with torch.cuda.stream(_error_word_stream(cuda, graph)):
        assert ops.decode_sync_status(cuda) == 0


def test_scheduler_client_raises_on_invalid_step(cuda):
    """The scheduler's model client reads every step's tokens: a step whose
    tokens are -1 raises there."""
    from lite_lang_amd.models.runner_batch import DecodeStepError
    from lite_lang_amd.scheduler.model_client import LocalModelClient
    ops = _ops()
    runner = _runner(cuda, True)
    client = LocalModelClient(runner)
    g = torch.Generator().manual_seed(5)
    msgs = [{"id": i, "input_tokens": torch.randint(0, 4096, (30 + i,), generator=g).tolist()}
            for i in range(4)]
    print("case: scheduler client invalid step", flush=True)
    client.add_batch(msgs, "c")
    client.prefill("c")
    client.decode("c")
    with torch.cuda.stream(_error_word_stream(cuda, True)):
        ops.decode_sync_error(cuda).fill_(1)
    torch.cuda.synchronize()
    with pytest.raises(DecodeStepError):
        client.decode("c")
    runner.reset_decode_fault()


def test_attention_merge_give_up_sets_error_word(cuda):
    """The fused decode attention's same-launch split merge waits for the
    other splits' partial words with a bound. In the spin limit's test mode
    (the merge never takes the words as written, 64 polls) every merge gives
    up: its rows come out NaN, the decode error word is set, and every kernel
    exits; the new token's K/V still reach the pool. After the word is reset
    and the attention workspace cleared (what Qwen2ModelRunner.reset_decode_fault
    does), the same call gives the default call's output bit for bit and
    leaves the workspace at zero."""
    from lite_lang_amd import _lib
    from tests.test_gpu_decode_rope_fused import _case, _fused
    ops = _ops()
    B, H, KVH, D, S, dt = 40, 16, 2, 128, 4, torch.bfloat16
    d, pool, max_len, _ = _case(cuda, B, H, KVH, D, [600] * B, S, dt, seed=12)
    assert 2 <= _lib.load().ll_decode_attention_split_count(B, KVH, D, max_len) <= 8
    print("case: attention merge gives up 40x16/2x128 len 600", flush=True)
    ops.decode_sync_status(cuda, reset=True)
    want, pool_want = _fused(cuda, d, pool, B, H, KVH, D, S, max_len, dt)
    torch.cuda.synchronize()
    assert ops.decode_sync_status(cuda) == 0
    ops.set_decode_spin_limit(-64)
    try:
        got, pool_got = _fused(cuda, d, pool, B, H, KVH, D, S, max_len, dt)
        torch.cuda.synchronize()
    finally:
        ops.set_decode_spin_limit(0)
    assert ops.decode_sync_status(cuda) == 1
    assert torch.isnan(got.float()).all()
    assert torch.equal(pool_got, pool_want)
    ops.decode_sync_status(cuda, reset=True)
    ops.clear_workspace(cuda, "decode_attention")
    again, _ = _fused(cuda, d, pool, B, H, KVH, D, S, max_len, dt)
    torch.cuda.synchronize()
    assert torch.equal(again, want)
    assert ops.decode_sync_status(cuda) == 0
    assert ops.workspace(cuda, "decode_attention", 0).count_nonzero() == 0


@pytest.mark.parametrize("shape", [(40, 12, 2, 128, [600] * 40), (7, 16, 2, 64, None)])
def test_split_merge_fallback_equals_same_launch(cuda, shape):
    """The runner's fallback when the XCD premise fails: with the same-launch
    merge switched off, decode attention merges its splits in a separate
    kernel; the outputs equal the same-launch merge's bit for bit (same
    partials, same combine arithmetic)."""
    ops = _ops()
    B, H, KVH, D, lens = shape
    rs = np.random.RandomState(6)
    if lens is None:
        lens = rs.randint(1, 3000, size=B).tolist()
    max_len = max(lens)
    P = B * max_len
    g = torch.Generator(device=cuda).manual_seed(6)
    q = torch.randn(B, H, D, device=cuda, generator=g).bfloat16()
    pool = torch.randn(P, 2 * KVH, D, device=cuda, generator=g).bfloat16()
    r2t = torch.from_numpy(rs.permutation(P).astype(np.int32)).view(B, max_len).to(cuda)
    rids = torch.arange(B, dtype=torch.int32, device=cuda)
    ln = torch.tensor(lens, dtype=torch.int64, device=cuda)
    print(f"case: merge fallback {B}x{H}/{KVH}x{D} max_len {max_len}", flush=True)
    assert ops.decode_attention_xcd_premise(cuda, B, H, KVH, D, max_len)
    a = torch.empty_like(q)
    ops.decode_attention(q, r2t, rids, ln, max_len, pool[:, :KVH], pool[:, KVH:], a)
    prev = ops.set_same_launch_merge(False)
    try:
        b = torch.empty_like(q)
        ops.decode_attention(q, r2t, rids, ln, max_len, pool[:, :KVH], pool[:, KVH:], b)
        torch.cuda.synchronize()
    finally:
        ops.set_same_launch_merge(prev)
    assert prev is True
    assert torch.equal(a, b)


def test_runner_checks_the_merge_premise(cuda):
    runner = _runner(cuda, True)
    print("case: runner merge premise", flush=True)
    assert runner.same_launch_merge is True
