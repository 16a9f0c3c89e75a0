"""Torch-tensor front end of the C ABI.

Every function here takes torch tensors that live on a HIP device, checks
shapes the way the reference does (Python ``assert``), and launches the
matching ``ll_*`` entry point on torch's current stream. Nothing here
computes on the host; a missing library raises at import.
"""
from __future__ import annotations

import torch

from . import _lib

_L = _lib.load()

_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_IDX = {torch.int32: 0, torch.int64: 1}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _idx(t: torch.Tensor, name: str) -> int:
    try:
        return _IDX[t.dtype]
    except KeyError:
        raise TypeError(f"{name}: index tensor must be int32 or int64, got {t.dtype}") from None


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("lite_lang_amd ops need device tensors (got a CPU tensor)")


# ------------------------------------------------------------------ workspaces
# Persistent, zero-initialised device buffers keyed by (device, stream, name).
# Tickets inside them are left at zero by the kernels, so they are zeroed only
# when a buffer is allocated.
#  * Per stream: work queued on two streams never shares a buffer, so a
#    second stream gets buffers of its own instead of racing on the first
#    one's. (Graphs are captured on torch's capture stream, so every captured
#    decode step shares that stream's set; replays of them are issued one
#    after another by the runner.)
#  * Never freed: a HIP graph keeps the raw addresses it was captured with,
#    so a buffer that grows is replaced by a larger one (twice the old size
#    at least) and the old one is kept alive in _RETIRED, where graphs
#    captured earlier still find it.
_WS: dict[tuple[int, int, str], torch.Tensor] = {}
_RETIRED: list[torch.Tensor] = []


def _ws_key(device: torch.device, name: str):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return (idx, torch.cuda.current_stream(idx).cuda_stream, name)


def workspace(device: torch.device, name: str, nbytes: int) -> torch.Tensor:
    key = _ws_key(device, name)
    buf = _WS.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None and torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"workspace '{name}' must be sized before graph capture")
        size = max(nbytes, 256)
        if buf is not None:
            size = max(size, 2 * buf.numel())
            _RETIRED.append(buf)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _WS[key] = buf
    return buf


def reserve_workspace(device: torch.device, name: str, nbytes: int) -> None:
    workspace(device, name, nbytes)


def clear_workspace(device: torch.device, name: str) -> None:
    """Zero the current stream's workspace `name`, if it exists."""
    buf = _WS.get(_ws_key(device, name))
    if buf is not None:
        buf.zero_()


# ------------------------------------------------------------------ attention
def decode_attention(q, req_to_tokens, b_req_idx, b_seq_len, max_len_in_batch, cache_k, cache_v,
                     out, sm_scale=None):
    """out[b, h] = softmax(q[b,h] K^T / sqrt(D)) V over the slot-table rows."""
    _dev(q, req_to_tokens, b_req_idx, b_seq_len, cache_k, cache_v, out)
    B, H, D = q.shape
    KVH = cache_k.shape[1]
    assert cache_k.shape[-1] == D and cache_v.shape[-1] == D
    assert q.stride(-1) == 1 and cache_k.stride(-1) == 1 and cache_v.stride(-1) == 1
    assert out.shape == q.shape and out.stride(-1) == 1
    assert H % KVH == 0
    if req_to_tokens.dtype != torch.int32:
        req_to_tokens = req_to_tokens.to(torch.int32)
    assert req_to_tokens.stride(-1) == 1
    if sm_scale is None:
        sm_scale = 1.0 / (D ** 0.5)
    max_len = int(max_len_in_batch)
    nbytes = _L.ll_decode_attention_workspace_size(B, H, KVH, D, max_len)
    ws = workspace(q.device, "decode_attention", nbytes)
    rc = _L.ll_decode_attention(
        q.data_ptr(), q.stride(0), q.stride(1),
        cache_k.data_ptr(), cache_k.stride(0), cache_k.stride(1),
        cache_v.data_ptr(), cache_v.stride(0), cache_v.stride(1),
        req_to_tokens.data_ptr(), req_to_tokens.stride(0),
        b_req_idx.data_ptr(), _idx(b_req_idx, "b_req_idx"),
        b_seq_len.data_ptr(), _idx(b_seq_len, "b_seq_len"),
        out.data_ptr(), out.stride(0), out.stride(1),
        B, H, KVH, D, max_len, float(sm_scale), dtype_code(q),
        ws.data_ptr(), ws.numel(), _stream(q))
    _lib.check(rc, "ll_decode_attention")
    return out


def decode_attention_xcd_premise(device, batch, q_heads, kv_heads, head_dim, max_len,
                                 launches=3):
    """Checks, on this machine, the premise of the split stage's own merge:
    the probe kernel runs on exactly the split stage's grid, block and LDS
    size for this shape and reports every workgroup's XCD; the premise holds
    when workgroups whose indices agree mod 8 ran on one XCD (the split stage
    gives every workgroup of a sequence indices of one residue), which the
    dispatcher's round-robin over 8 XCDs gives, and so does a device of one
    XCD. Returns True/False (True when the shape runs no split stage: head
    dims other than 64/128)."""
    if head_dim not in (64, 128) or batch <= 0 or q_heads % kv_heads != 0:
        return True
    cap = 1 << 16
    out = torch.full((cap,), -1, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    for _ in range(launches):
        n = _L.ll_decode_attention_xcc_probe(batch, q_heads, kv_heads, head_dim, max_len,
                                             out.data_ptr(), cap, stream)
        if n < 0:
            _lib.check(n, "ll_decode_attention_xcc_probe")
        got = out[:n].cpu().long()
        if int(got.min()) < 0:
            return False
        # workgroup i against workgroup i mod 8
        if not bool(torch.all(got == got[torch.arange(n) % 8])):
            return False
    return True


def set_same_launch_merge(enable):
    """Process-wide: whether decode attention merges its splits in the split
    stage (default) or in a separate kernel; returns the previous setting."""
    return bool(_L.ll_decode_attention_set_same_launch_merge(int(bool(enable))))


def prefill_attention(q, k, v, o, b_req_idx, b_start_loc, b_seq_len, max_input_len,
                      req_to_tokens, b_shared_seq_len=None, sm_scale=None):
    """NoPad causal prefill over the slot table (optionally with shared prefixes)."""
    _dev(q, k, v, o, b_req_idx, b_start_loc, b_seq_len, req_to_tokens)
    T, H, D = q.shape
    KVH = k.shape[1]
    assert k.shape[-1] == D and v.shape[-1] == D
    assert q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1 and o.stride(-1) == 1
    assert H % KVH == 0
    if req_to_tokens.dtype != torch.int32:
        req_to_tokens = req_to_tokens.to(torch.int32)
    if sm_scale is None:
        sm_scale = 1.0 / (D ** 0.5)
    B = b_seq_len.shape[0]
    sh_ptr, sh64 = (0, 0)
    if b_shared_seq_len is not None:
        _dev(b_shared_seq_len)
        sh_ptr, sh64 = b_shared_seq_len.data_ptr(), _idx(b_shared_seq_len, "b_shared_seq_len")
    rc = _L.ll_prefill_attention(
        q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        o.data_ptr(), o.stride(0), o.stride(1),
        req_to_tokens.data_ptr(), req_to_tokens.stride(0),
        b_req_idx.data_ptr(), _idx(b_req_idx, "b_req_idx"),
        b_start_loc.data_ptr(), _idx(b_start_loc, "b_start_loc"),
        b_seq_len.data_ptr(), _idx(b_seq_len, "b_seq_len"),
        sh_ptr or None, sh64,
        B, H, KVH, D, int(max_input_len), float(sm_scale), dtype_code(q), _stream(q))
    _lib.check(rc, "ll_prefill_attention")
    return o


# ------------------------------------------------------------------ elementwise
def rmsnorm(x, gamma, eps, residual=None, out=None):
    """out = rmsnorm(x [+ residual]) * gamma; with residual, x is updated in place."""
    _dev(x, gamma, residual, out)
    assert x.ndim == 2 and x.shape[1] == gamma.shape[0]
    assert x.stride(1) == 1 and gamma.stride(0) == 1
    if out is None:
        out = torch.empty_like(x)
    assert out.shape == x.shape and out.stride(1) == 1
    r_ptr, r_rs = (None, 0)
    if residual is not None:
        assert residual.shape == x.shape and residual.stride(1) == 1
        r_ptr, r_rs = residual.data_ptr(), residual.stride(0)
    rc = _L.ll_rmsnorm(x.data_ptr(), x.stride(0), r_ptr, r_rs, gamma.data_ptr(), out.data_ptr(),
                       out.stride(0), x.shape[0], x.shape[1], float(eps), dtype_code(x),
                       _stream(x))
    _lib.check(rc, "ll_rmsnorm")
    return out


def rotary_emb(q, k, cos, sin):
    _dev(q, k, cos, sin)
    T, Hq, D = q.shape
    Hk = k.shape[1]
    assert q.stride(2) == 1 and k.stride(2) == 1 and cos.stride(1) == 1 and sin.stride(1) == 1
    assert cos.dtype == sin.dtype
    rc = _L.ll_rotary_emb(q.data_ptr(), q.stride(0), q.stride(1), Hq,
                          k.data_ptr(), k.stride(0), k.stride(1), Hk,
                          cos.data_ptr(), cos.stride(0), sin.data_ptr(), sin.stride(0),
                          T, D, dtype_code(q), dtype_code(cos), _stream(q))
    _lib.check(rc, "ll_rotary_emb")


def rope_kv_scatter(qkv, q_heads, kv_heads, head_dim, positions, cos_table, sin_table, slots,
                    pool_layer):
    """Rotate q in place inside qkv; write rotated K and V to pool_layer[slots]."""
    _dev(qkv, positions, cos_table, sin_table, slots, pool_layer)
    T = qkv.shape[0]
    assert qkv.stride(1) == 1 and qkv.shape[1] == (q_heads + 2 * kv_heads) * head_dim
    assert slots.dtype == torch.int32 and pool_layer.stride(-1) == 1
    assert cos_table.stride(1) == 1 and cos_table.stride(0) == sin_table.stride(0)
    rc = _L.ll_rope_kv_scatter(qkv.data_ptr(), qkv.stride(0), T, q_heads, kv_heads, head_dim,
                               positions.data_ptr(), _idx(positions, "positions"),
                               cos_table.data_ptr(), sin_table.data_ptr(), cos_table.stride(0),
                               dtype_code(cos_table), slots.data_ptr(), pool_layer.data_ptr(),
                               pool_layer.stride(0), pool_layer.stride(1), dtype_code(qkv),
                               _stream(qkv))
    _lib.check(rc, "ll_rope_kv_scatter")


def kv_store(src, slots, pool):
    _dev(src, slots, pool)
    T, Hs, D = src.shape
    assert slots.dtype == torch.int32 and src.stride(2) == 1 and pool.stride(-1) == 1
    rc = _L.ll_kv_store(src.data_ptr(), src.stride(0), src.stride(1), Hs, D, slots.data_ptr(),
                        pool.data_ptr(), pool.stride(0), pool.stride(1), T, dtype_code(src),
                        _stream(src))
    _lib.check(rc, "ll_kv_store")


def silu_and_mul(x, out=None):
    _dev(x, out)
    M, N2 = x.shape
    N = N2 // 2
    assert x.stride(1) == 1
    if out is None:
        out = x[:, :N]
    assert out.stride(1) == 1
    rc = _L.ll_silu_and_mul(x.data_ptr(), x.stride(0), out.data_ptr(), out.stride(0), M, N,
                            dtype_code(x), _stream(x))
    _lib.check(rc, "ll_silu_and_mul")
    return out


def embedding(table, ids, out=None):
    _dev(table, ids, out)
    V, Hd = table.shape
    T = ids.shape[0]
    assert table.stride(1) == 1
    if out is None:
        out = torch.empty((T, Hd), dtype=table.dtype, device=table.device)
    rc = _L.ll_embedding(table.data_ptr(), table.stride(0), V, ids.data_ptr(), _idx(ids, "ids"),
                         out.data_ptr(), out.stride(0), T, Hd, dtype_code(table), _stream(table))
    _lib.check(rc, "ll_embedding")
    return out


def embedding_rmsnorm(table, ids, gamma, eps, epoch=None, slot_write=None):
    """(h, out): h = table[ids], out = rmsnorm(h) * gamma, in one launch. With
    `epoch` (the int32 word of decode_epoch), the launch also adds 1 to it;
    with slot_write = (req_to_tokens, packed) (and epoch), it also does
    assign_slots(req_to_tokens, packed, len(ids))."""
    _dev(table, ids, gamma, epoch)
    V, Hd = table.shape
    T = ids.shape[0]
    assert table.stride(1) == 1 and gamma.shape == (Hd,)
    h = torch.empty((T, Hd), dtype=table.dtype, device=table.device)
    out = torch.empty_like(h)
    head = (table.data_ptr(), table.stride(0), V, ids.data_ptr(), _idx(ids, "ids"), h.data_ptr(),
            h.stride(0), gamma.data_ptr(), out.data_ptr(), out.stride(0), T, Hd, float(eps),
            dtype_code(table))
    if epoch is None:
        assert slot_write is None, "embedding_rmsnorm: slot_write needs the epoch form"
        rc = _L.ll_embedding_rmsnorm(*head, _stream(table))
    else:
        assert epoch.dtype == torch.int32 and epoch.numel() == 1
        sw = (None, 0, None, None, None)
        if slot_write is not None:
            r2t, packed = slot_write
            _dev(r2t, packed)
            assert r2t.dtype == torch.int32 and r2t.stride(1) == 1
            assert packed.dtype == torch.int32 and packed.shape[0] == 3 and packed.shape[1] >= T
            sw = (r2t.data_ptr(), r2t.stride(0), packed[0].data_ptr(), packed[1].data_ptr(),
                  packed[2].data_ptr())
        rc = _L.ll_embedding_rmsnorm_epoch(*head, epoch.data_ptr(), *sw, _stream(table))
    _lib.check(rc, "ll_embedding_rmsnorm")
    return h, out


def argmax(x, out=None, status=None):
    """First-index argmax of every row; with `status` (an int32 device word,
    decode_sync_error's), every output is -1 while that word is nonzero."""
    _dev(x, out, status)
    M, N = x.shape
    assert x.stride(1) == 1
    if out is None:
        out = torch.empty((M,), dtype=torch.int64, device=x.device)
    nbytes = _L.ll_argmax_workspace_size(M, N)
    ws = workspace(x.device, "argmax", nbytes)
    head = (x.data_ptr(), x.stride(0), M, N, out.data_ptr(), ws.data_ptr(), ws.numel(),
            dtype_code(x))
    if status is None:
        rc = _L.ll_argmax(*head, _stream(x))
    else:
        rc = _L.ll_argmax_status(*head, status.data_ptr(), _stream(x))
    _lib.check(rc, "ll_argmax")
    return out


# ------------------------------------------------------------------ GEMM
def gemm(x, w, bias=None, out=None):
    """out[M, N] = x[M, K] @ w[N, K]^T (+ bias); w in nn.Linear [out, in] layout."""
    _dev(x, w, bias, out)
    M, K = x.shape
    N, K2 = w.shape
    assert K == K2, f"gemm: K mismatch {K} vs {K2}"
    assert x.stride(1) == 1 and w.stride(1) == 1 and x.dtype == w.dtype
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    assert out.shape == (M, N) and out.stride(1) == 1
    nbytes = _L.ll_gemm_workspace_size(M, N, K)
    ws_ptr, ws_n = (None, 0)
    if nbytes > 0:
        ws = workspace(x.device, "gemm", nbytes)
        ws_ptr, ws_n = ws.data_ptr(), ws.numel()
    rc = _L.ll_gemm(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                    bias.data_ptr() if bias is not None else None, out.data_ptr(), out.stride(0),
                    M, N, K, dtype_code(x), ws_ptr, ws_n, _stream(x))
    _lib.check(rc, "ll_gemm")
    return out


def gemm_tiled(x, w, bias=None, out=None):
    """out[M, N] = x @ w^T (+ bias) on the 256 x 256 MFMA tile kernel (prefill)."""
    _dev(x, w, bias, out)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape[1] == K and x.stride(1) == 1 and w.stride(1) == 1 and x.dtype == w.dtype
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    assert out.shape == (M, N) and out.stride(1) == 1
    rc = _L.ll_gemm_tiled(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                          bias.data_ptr() if bias is not None else None, out.data_ptr(),
                          out.stride(0), M, N, K, dtype_code(x), _stream(x))
    _lib.check(rc, "ll_gemm_tiled")
    return out


def gemm_tiled_supported(M, N, K, dtype) -> bool:
    return dtype in (torch.bfloat16, torch.float16) and bool(
        _L.ll_gemm_tiled_supported(M, N, K, _DTYPES[dtype]))


def interleave_gate_up(w):
    """[gate; up] weight [2I, K] (16-bit or int8) -> the 64-row interleaved copy
    the fused gate/up + SiLU tile kernels read, or None when I % 128 != 0."""
    _dev(w)
    N2, K = w.shape
    I = N2 // 2
    es = w.element_size()
    if N2 % 2 or I % 128 or (K * es) % 16 or w.stride(1) != 1:
        return None
    out = torch.empty_like(w, memory_format=torch.contiguous_format)
    rc = _L.ll_gemm_interleave_gate_up(w.data_ptr(), w.stride(0), I, K, es, out.data_ptr(),
                                       _stream(w))
    _lib.check(rc, "ll_gemm_interleave_gate_up")
    return out


def gate_up_silu_tiled(x, w_il, out=None):
    """silu(x @ gate^T) * (x @ up^T) from the interleaved weight (prefill)."""
    _dev(x, w_il, out)
    M, K = x.shape
    I = w_il.shape[0] // 2
    assert w_il.shape[1] == K and x.stride(1) == 1 and x.dtype == w_il.dtype
    if out is None:
        out = torch.empty((M, I), dtype=x.dtype, device=x.device)
    assert out.shape == (M, I) and out.stride(1) == 1
    rc = _L.ll_gemm_gate_up_silu_tiled(x.data_ptr(), x.stride(0), w_il.data_ptr(), M, I, K,
                                       dtype_code(x), out.data_ptr(), out.stride(0), _stream(x))
    _lib.check(rc, "ll_gemm_gate_up_silu_tiled")
    return out


def gemm_i8_tiled(xq, s_tok, wq, s_ch, bias=None, out_dtype=torch.bfloat16, out=None):
    """dequantised W8A8 product out[M, N] (prefill tile kernel)."""
    _dev(xq, s_tok, wq, s_ch, bias, out)
    M, K = xq.shape
    N = wq.shape[0]
    assert wq.shape[1] == K and xq.dtype == torch.int8 and wq.dtype == torch.int8
    assert s_tok.dtype == torch.float32 and s_ch.numel() == N
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=xq.device)
    rc = _L.ll_gemm_i8_tiled(xq.data_ptr(), xq.stride(0), s_tok.data_ptr(), wq.data_ptr(),
                             wq.stride(0), s_ch.data_ptr(), dtype_code(s_ch),
                             bias.data_ptr() if bias is not None else None, out.data_ptr(),
                             out.stride(0), M, N, K, dtype_code(out), _stream(xq))
    _lib.check(rc, "ll_gemm_i8_tiled")
    return out


def gemm_i8_i32_tiled(xq, wq, out=None):
    """exact int32 sums int8(x) @ int8(w)^T on the prefill tile kernel."""
    _dev(xq, wq, out)
    M, K = xq.shape
    N = wq.shape[0]
    assert wq.shape[1] == K and xq.dtype == torch.int8 and wq.dtype == torch.int8
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32, device=xq.device)
    rc = _L.ll_gemm_i8_i32_tiled(xq.data_ptr(), xq.stride(0), wq.data_ptr(), wq.stride(0),
                                 out.data_ptr(), out.stride(0), M, N, K, _stream(xq))
    _lib.check(rc, "ll_gemm_i8_i32_tiled")
    return out


def gemm_i8_i32(xq, wq, out=None):
    """exact int32 sums int8(x) @ int8(w)^T for any shape (the tile kernel
    where its layout holds, else a plain dot-product kernel)."""
    _dev(xq, wq, out)
    M, K = xq.shape
    N = wq.shape[0]
    assert wq.shape[1] == K and xq.dtype == torch.int8 and wq.dtype == torch.int8
    assert xq.stride(1) == 1 and wq.stride(1) == 1
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32, device=xq.device)
    assert out.shape == (M, N) and out.stride(1) == 1 and out.dtype == torch.int32
    rc = _L.ll_gemm_i8_i32(xq.data_ptr(), xq.stride(0), wq.data_ptr(), wq.stride(0),
                           out.data_ptr(), out.stride(0), M, N, K, _stream(xq))
    _lib.check(rc, "ll_gemm_i8_i32")
    return out


def gemm_i8_tiled_supported(M, N, K) -> bool:
    """Shapes the int8 tile kernel takes (K % 64 == 0, N % 4 == 0)."""
    return M > 0 and N % 4 == 0 and K % 64 == 0


def gemm_i8_gate_up_silu_tiled(xq, s_tok, wq_il, s_ch, out_dtype=torch.bfloat16, out=None):
    """W8A8 gate/up + SiLU_and_Mul from the interleaved int8 weight (prefill)."""
    _dev(xq, s_tok, wq_il, s_ch, out)
    M, K = xq.shape
    I = wq_il.shape[0] // 2
    if out is None:
        out = torch.empty((M, I), dtype=out_dtype, device=xq.device)
    rc = _L.ll_gemm_i8_gate_up_silu_tiled(xq.data_ptr(), xq.stride(0), s_tok.data_ptr(),
                                          wq_il.data_ptr(), s_ch.data_ptr(), dtype_code(s_ch),
                                          M, I, K, dtype_code(out), out.data_ptr(), out.stride(0),
                                          _stream(xq))
    _lib.check(rc, "ll_gemm_i8_gate_up_silu_tiled")
    return out


# ------------------------------------------------------------------ slot table
def assign_slots(req_to_tokens, packed, n):
    """req_to_tokens[rows, cols] = slots with packed = int32 [3, n] (slots, rows, cols)."""
    _dev(req_to_tokens, packed)
    assert req_to_tokens.dtype == torch.int32 and packed.dtype == torch.int32
    assert packed.is_contiguous() and packed.shape[0] == 3
    rc = _L.ll_assign_slots(req_to_tokens.data_ptr(), req_to_tokens.stride(0), packed[0].data_ptr(),
                            packed[1].data_ptr(), packed[2].data_ptr(), n, _stream(req_to_tokens))
    _lib.check(rc, "ll_assign_slots")


# ------------------------------------------------------------------ decode split-K path
def gemm_splitk_count(M, N, K) -> int:
    return _L.ll_gemm_splitk_count(M, N, K)


def gemm_splitk(x, w, part):
    """fp32 partial sums of x[M, K] @ w[N, K]^T into part (flat fp32 buffer);
    returns the split count s (part[:s*M*N] holds [s, M, N])."""
    _dev(x, w, part)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape[1] == K and x.stride(1) == 1 and w.stride(1) == 1 and part.dtype == torch.float32
    s = _L.ll_gemm_splitk_count(M, N, K)
    rc = _L.ll_gemm_splitk(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), M, N, K,
                           dtype_code(x), part.data_ptr(), part.numel() * 4, _stream(x))
    _lib.check(rc, "ll_gemm_splitk")
    return s


class PackedWeight:
    """A [N, K] nn.Linear weight in the weight-streaming kernel's packed layout
    (ll_gemm_pack); keeps the logical shape next to the packed bytes."""

    def __init__(self, w):
        _dev(w)
        N, K = w.shape
        assert w.stride(1) == 1 and w.dtype in (torch.bfloat16, torch.float16)
        nbytes = _L.ll_gemm_packed_bytes(N, K)
        if nbytes <= 0:
            raise _lib.LiteLangError(f"ll_gemm_pack: K={K} is not a multiple of 128")
        self.shape, self.dtype, self.device = (N, K), w.dtype, w.device
        self.data = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
        rc = _L.ll_gemm_pack(w.data_ptr(), w.stride(0), N, K, dtype_code(w), self.data.data_ptr(),
                             nbytes, _stream(w))
        _lib.check(rc, "ll_gemm_pack")


class PackedGateUp:
    """[gate; up] weight ([2I, K]) packed for the fused gate/up + SiLU_and_Mul GEMM."""

    def __init__(self, w):
        _dev(w)
        N2, K = w.shape
        assert N2 % 2 == 0 and w.stride(1) == 1 and w.dtype in (torch.bfloat16, torch.float16)
        I = N2 // 2
        nbytes = _L.ll_gemm_packed_gate_up_bytes(I, K)
        if nbytes <= 0:
            raise _lib.LiteLangError(f"ll_gemm_pack_gate_up: K={K} is not a multiple of 128")
        self.shape, self.inter, self.dtype, self.device = (N2, K), I, w.dtype, w.device
        self.data = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
        rc = _L.ll_gemm_pack_gate_up(w.data_ptr(), w.stride(0), I, K, dtype_code(w),
                                     self.data.data_ptr(), nbytes, _stream(w))
        _lib.check(rc, "ll_gemm_pack_gate_up")


def pack_gate_up(w):
    """Packed [gate; up] weight for gate_up_silu, or None when K % 128 != 0."""
    if w.dtype not in (torch.bfloat16, torch.float16) or w.shape[1] % 128 != 0:
        return None
    return PackedGateUp(w)


def gate_up_silu(x, wp: PackedGateUp, out=None):
    """silu(x @ gate^T) * (x @ up^T) for M <= 64, rounded as silu_and_mul_splitk."""
    _dev(x, out)
    M, K = x.shape
    assert wp.shape[1] == K and x.stride(1) == 1 and x.dtype == wp.dtype
    if out is None:
        out = torch.empty((M, wp.inter), dtype=x.dtype, device=x.device)
    assert out.shape == (M, wp.inter) and out.stride(1) == 1
    rc = _L.ll_gemm_gate_up_silu_packed(x.data_ptr(), x.stride(0), wp.data.data_ptr(), M, wp.inter,
                                        K, dtype_code(x), out.data_ptr(), out.stride(0), _stream(x))
    _lib.check(rc, "ll_gemm_gate_up_silu_packed")
    return out


def pack_weight(w):
    """Packed copy of w for gemm_splitk / gemm with M <= 64, or None when K % 128 != 0."""
    if w.dtype not in (torch.bfloat16, torch.float16) or w.shape[1] % 128 != 0:
        return None
    return PackedWeight(w)


def gemm_splitk_packed(x, wp: PackedWeight, part):
    """gemm_splitk with a packed weight; returns the split count."""
    _dev(x, part)
    M, K = x.shape
    N = wp.shape[0]
    assert wp.shape[1] == K and x.stride(1) == 1 and x.dtype == wp.dtype
    assert part.dtype == torch.float32
    s = _L.ll_gemm_splitk_count(M, N, K)
    rc = _L.ll_gemm_splitk_packed(x.data_ptr(), x.stride(0), wp.data.data_ptr(), M, N, K,
                                  dtype_code(x), part.data_ptr(), part.numel() * 4, _stream(x))
    _lib.check(rc, "ll_gemm_splitk_packed")
    return s


def gemm_packed_argmax(x, wp: PackedWeight, logits=None, out=None, status=None):
    """The fp32 logits x @ w^T (M <= 64, packed weight) and their first-index
    argmax in one call (ll_gemm_packed_f32_argmax); with `status`, every token
    is -1 while that word is nonzero. Returns (logits, tokens)."""
    _dev(x, logits, out, status)
    M, K = x.shape
    N = wp.shape[0]
    assert wp.shape[1] == K and x.stride(1) == 1 and x.dtype == wp.dtype
    if logits is None:
        logits = torch.empty((M, N), dtype=torch.float32, device=x.device)
    if out is None:
        out = torch.empty((M,), dtype=torch.int64, device=x.device)
    assert logits.shape == (M, N) and logits.stride(1) == 1 and logits.dtype == torch.float32
    assert out.numel() == M and out.dtype == torch.int64 and out.is_contiguous()
    nbytes = _L.ll_gemm_packed_f32_argmax_workspace_size(M, N, K)
    ws = workspace(x.device, "lm_argmax", nbytes)
    rc = _L.ll_gemm_packed_f32_argmax(x.data_ptr(), x.stride(0), wp.data.data_ptr(), None,
                                      logits.data_ptr(), logits.stride(0), M, N, K, dtype_code(x),
                                      out.data_ptr(),
                                      status.data_ptr() if status is not None else None,
                                      ws.data_ptr(), ws.numel(), _stream(x))
    _lib.check(rc, "ll_gemm_packed_f32_argmax")
    return logits, out


def gemm_packed(x, wp: PackedWeight, bias=None, out=None, out_dtype=None):
    """out[M, N] = x @ w^T (+ bias) for M <= 64 from a packed weight; with
    out_dtype=torch.float32 the sums are written unrounded (fp32)."""
    _dev(x, bias, out)
    M, K = x.shape
    N = wp.shape[0]
    assert wp.shape[1] == K and x.stride(1) == 1 and x.dtype == wp.dtype
    out_dtype = out_dtype or (out.dtype if out is not None else x.dtype)
    assert out_dtype in (x.dtype, torch.float32)
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    assert out.shape == (M, N) and out.stride(1) == 1 and out.dtype == out_dtype
    nbytes = _L.ll_gemm_workspace_size(M, N, K)
    ws_ptr, ws_n = (None, 0)
    if nbytes > 0:
        ws = workspace(x.device, "gemm", nbytes)
        ws_ptr, ws_n = ws.data_ptr(), ws.numel()
    fn = _L.ll_gemm_packed_f32 if out_dtype == torch.float32 else _L.ll_gemm_packed
    rc = fn(x.data_ptr(), x.stride(0), wp.data.data_ptr(),
            bias.data_ptr() if bias is not None else None, out.data_ptr(),
            out.stride(0), M, N, K, dtype_code(x), ws_ptr, ws_n, _stream(x))
    _lib.check(rc, "ll_gemm_packed")
    return out


def add_rmsnorm_splitk(h, part, splits, gamma, eps, out=None):
    """h = dtype(h + dtype(sum part)); returns rmsnorm(h) * gamma."""
    _dev(h, part, gamma, out)
    M, N = h.shape
    if out is None:
        out = torch.empty_like(h)
    rc = _L.ll_add_rmsnorm_splitk(h.data_ptr(), h.stride(0), part.data_ptr(), splits,
                                  gamma.data_ptr(), out.data_ptr(), out.stride(0), M, N, float(eps),
                                  dtype_code(h), _stream(h))
    _lib.check(rc, "ll_add_rmsnorm_splitk")
    return out


def add_rmsnorm_qkv_splits(M, hidden, nqkv):
    """k splits of add_rmsnorm_qkv_splitk's QKV partials; 0 when the shape is
    not covered (then run add_rmsnorm_splitk and the split-K GEMM)."""
    return int(_L.ll_add_rmsnorm_qkv_splits(M, hidden, nqkv))


def decode_sync(device):
    """The flag words of the fused decode launches on the current stream."""
    return workspace(device, "decode_sync", int(_L.ll_decode_sync_bytes()))


def decode_epoch(device):
    """The decode-step epoch word of the current stream (int32 [1]): every
    fused launch of one step uses it with its own tag, and the step's first
    launch advances it (embedding_rmsnorm(epoch=...))."""
    return workspace(device, "decode_epoch", 4).view(torch.int32)[:1]


def decode_epoch_advance(device):
    """Advance the decode-step epoch word with a launch of its own (a
    device-side add, so a captured graph advances it on every replay) and
    return it; the model's decode step advances it inside its first launch
    instead."""
    ep = decode_epoch(device)
    ep.add_(1)
    return ep


def decode_sync_error(device):
    """The error word of the current stream's decode sync words (int32 [1]):
    nonzero once a fused launch's flag wait gave up, until reset."""
    off = int(_L.ll_decode_sync_error_offset())
    return decode_sync(device)[off:off + 4].view(torch.int32)


def set_decode_spin_limit(polls):
    """Polls before a fused launch's flag wait gives up (0: the default)."""
    _lib.check(_L.ll_decode_sync_set_spin_limit(int(polls)), "ll_decode_sync_set_spin_limit")


def decode_sync_status(device, reset=False):
    """1 when a fused launch's flag wait gave up (its outputs are invalid)."""
    sync = decode_sync(device)
    rc = _L.ll_decode_sync_status(sync.data_ptr(), int(bool(reset)),
                                  torch.cuda.current_stream(device).cuda_stream)
    if rc < 0:
        _lib.check(rc, "ll_decode_sync_status")
    return rc


def add_rmsnorm_qkv_splitk(h, part, splits, gamma, eps, wp: PackedWeight, qkv_part, epoch, tag,
                           x=None):
    """h = dtype(h + dtype(sum part)); x = rmsnorm(h) * gamma (as
    add_rmsnorm_splitk), and the QKV split-K partials of x @ w^T into
    qkv_part (may be part) in the same launch. Returns (x, qkv splits)."""
    _dev(h, part, gamma, qkv_part, epoch, x)
    M, hidden = h.shape
    nqkv = wp.shape[0]
    assert wp.shape[1] == hidden and wp.dtype == h.dtype and h.stride(1) == 1
    assert part.dtype == torch.float32 and qkv_part.dtype == torch.float32
    assert epoch.dtype == torch.int32 and 0 <= int(tag) < 256
    qs = add_rmsnorm_qkv_splits(M, hidden, nqkv)
    if qs <= 0:
        raise _lib.LiteLangError(f"add_rmsnorm_qkv_splitk: shape not covered (M={M} "
                                 f"hidden={hidden} nqkv={nqkv})")
    if x is None:
        x = torch.empty((M, hidden), dtype=h.dtype, device=h.device)
    assert x.shape == (M, hidden) and x.is_contiguous()
    sync = decode_sync(h.device)
    rc = _L.ll_add_rmsnorm_qkv_splitk(h.data_ptr(), h.stride(0), part.data_ptr(), splits,
                                      gamma.data_ptr(), float(eps), x.data_ptr(),
                                      wp.data.data_ptr(), qkv_part.data_ptr(),
                                      qkv_part.numel() * 4, M, hidden, nqkv, dtype_code(h),
                                      sync.data_ptr(), epoch.data_ptr(), int(tag), _stream(h))
    _lib.check(rc, "ll_add_rmsnorm_qkv_splitk")
    return x, qs


def silu_and_mul_splitk(part, splits, out):
    """out[M, N] = up * dtype(silu(gate)) from partials of the [M, 2N] product."""
    _dev(part, out)
    M, N = out.shape
    rc = _L.ll_silu_and_mul_splitk(part.data_ptr(), splits, out.data_ptr(), out.stride(0), M, N,
                                   dtype_code(out), _stream(out))
    _lib.check(rc, "ll_silu_and_mul_splitk")
    return out


def rope_kv_scatter_splitk(part, splits, bias, q_out, q_heads, kv_heads, head_dim, positions,
                           cos_table, sin_table, slots, pool_layer):
    _dev(part, q_out, positions, cos_table, sin_table, slots, pool_layer)
    T = q_out.shape[0]
    assert slots.dtype == torch.int32 and q_out.stride(1) == 1 and pool_layer.stride(-1) == 1
    rc = _L.ll_rope_kv_scatter_splitk(
        part.data_ptr(), splits, bias.data_ptr() if bias is not None else None, q_out.data_ptr(),
        q_out.stride(0), T, q_heads, kv_heads, head_dim, positions.data_ptr(),
        _idx(positions, "positions"), cos_table.data_ptr(), sin_table.data_ptr(),
        cos_table.stride(0), dtype_code(cos_table), slots.data_ptr(), pool_layer.data_ptr(),
        pool_layer.stride(0), pool_layer.stride(1), dtype_code(q_out), _stream(q_out))
    _lib.check(rc, "ll_rope_kv_scatter_splitk")


def decode_attention_rope_splitk(part, splits, bias, positions, cos_table, sin_table, slots,
                                 req_to_tokens, b_req_idx, b_seq_len, max_len_in_batch, cache_k,
                                 cache_v, out, sm_scale=None):
    """rope_kv_scatter_splitk + decode_attention in one launch: q is rebuilt
    from the QKV split-K partials inside the attention kernel and the new
    token's K/V are written to cache_k/cache_v[slots[b]] by the workgroup that
    attends over that token. A split merge that gives up its bounded wait
    sets the current stream's decode error word (decode_sync_error)."""
    _dev(part, positions, cos_table, sin_table, slots, req_to_tokens, b_req_idx, b_seq_len,
         cache_k, cache_v, out)
    B, H, D = out.shape
    KVH = cache_k.shape[1]
    assert slots.dtype == torch.int32 and req_to_tokens.dtype == torch.int32
    assert cache_k.stride(-1) == 1 and cache_v.stride(-1) == 1 and out.stride(-1) == 1
    assert req_to_tokens.stride(-1) == 1 and cos_table.dtype == torch.float32
    if sm_scale is None:
        sm_scale = 1.0 / (D ** 0.5)
    max_len = int(max_len_in_batch)
    nbytes = _L.ll_decode_attention_workspace_size(B, H, KVH, D, max_len)
    ws = workspace(out.device, "decode_attention", nbytes)
    rc = _L.ll_decode_attention_rope_splitk(
        part.data_ptr(), splits, bias.data_ptr() if bias is not None else None,
        positions.data_ptr(), _idx(positions, "positions"), cos_table.data_ptr(),
        sin_table.data_ptr(), cos_table.stride(0), dtype_code(cos_table), slots.data_ptr(),
        cache_k.data_ptr(), cache_k.stride(0), cache_k.stride(1),
        cache_v.data_ptr(), cache_v.stride(0), cache_v.stride(1),
        req_to_tokens.data_ptr(), req_to_tokens.stride(0),
        b_req_idx.data_ptr(), _idx(b_req_idx, "b_req_idx"),
        b_seq_len.data_ptr(), _idx(b_seq_len, "b_seq_len"),
        out.data_ptr(), out.stride(0), out.stride(1),
        B, H, KVH, D, max_len, float(sm_scale), dtype_code(out), ws.data_ptr(), ws.numel(),
        decode_sync_error(out.device).data_ptr(), _stream(out))
    _lib.check(rc, "ll_decode_attention_rope_splitk")
    return out


def decode_attention_rope_splitk_i32(p, bias, positions, cos_table, sin_table, slots,
                                     req_to_tokens, b_req_idx, b_seq_len, max_len_in_batch,
                                     cache_k, cache_v, out, sm_scale=None, quant=False,
                                     input_scale=None):
    """decode_attention_rope_splitk from the int8 QKV projection's int32
    partials (an I8Partials), dequantised inline. With quant, also returns
    the output rows' int8 codes and scales for the o_proj (per token, or
    static with input_scale)."""
    _dev(p.part, positions, cos_table, sin_table, slots, req_to_tokens, b_req_idx, b_seq_len,
         cache_k, cache_v, out)
    B, H, D = out.shape
    KVH = cache_k.shape[1]
    assert slots.dtype == torch.int32 and req_to_tokens.dtype == torch.int32
    assert cache_k.stride(-1) == 1 and cache_v.stride(-1) == 1 and out.stride(-1) == 1
    assert req_to_tokens.stride(-1) == 1 and cos_table.dtype == torch.float32
    if sm_scale is None:
        sm_scale = 1.0 / (D ** 0.5)
    max_len = int(max_len_in_batch)
    nbytes = _L.ll_decode_attention_workspace_size(B, H, KVH, D, max_len)
    ws = workspace(out.device, "decode_attention", nbytes)
    q = torch.empty((B, H * D), dtype=torch.int8, device=out.device) if quant else None
    s = torch.empty((B,), dtype=torch.float32, device=out.device) if quant else None
    rc = _L.ll_decode_attention_rope_splitk_i32(
        p.part.data_ptr(), p.splits, p.s_tok.data_ptr(), p.s_ch.data_ptr(), dtype_code(p.s_ch),
        bias.data_ptr() if bias is not None else None,
        positions.data_ptr(), _idx(positions, "positions"), cos_table.data_ptr(),
        sin_table.data_ptr(), cos_table.stride(0), dtype_code(cos_table), slots.data_ptr(),
        cache_k.data_ptr(), cache_k.stride(0), cache_k.stride(1),
        cache_v.data_ptr(), cache_v.stride(0), cache_v.stride(1),
        req_to_tokens.data_ptr(), req_to_tokens.stride(0),
        b_req_idx.data_ptr(), _idx(b_req_idx, "b_req_idx"),
        b_seq_len.data_ptr(), _idx(b_seq_len, "b_seq_len"),
        out.data_ptr(), out.stride(0), out.stride(1),
        B, H, KVH, D, max_len, float(sm_scale), dtype_code(out), ws.data_ptr(), ws.numel(),
        input_scale.data_ptr() if input_scale is not None else None,
        q.data_ptr() if quant else None, H * D, s.data_ptr() if quant else None,
        decode_sync_error(out.device).data_ptr(), _stream(out))
    _lib.check(rc, "ll_decode_attention_rope_splitk_i32")
    return (out, q, s) if quant else out


# ------------------------------------------------------------------ W8A8
def quant_weight_per_channel(w):
    """(int8 [N, K], scale [N] in w's dtype): smooth_quant/layer.py:5-16 on the float path."""
    _dev(w)
    N, K = w.shape
    assert w.stride(1) == 1
    q = torch.empty((N, K), dtype=torch.int8, device=w.device)
    s = torch.empty((N,), dtype=w.dtype, device=w.device)
    rc = _L.ll_quant_weight_per_channel(w.data_ptr(), w.stride(0), N, K, dtype_code(w),
                                        q.data_ptr(), K, s.data_ptr(), _stream(w))
    _lib.check(rc, "ll_quant_weight_per_channel")
    return q, s


def quant_per_token(x, q=None, s=None):
    """(int8 [M, K], fp32 scale [M]): dynamic per-token absmax quantisation."""
    _dev(x, q, s)
    M, K = x.shape
    assert x.stride(1) == 1
    if q is None:
        q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if s is None:
        s = torch.empty((M,), dtype=torch.float32, device=x.device)
    rc = _L.ll_quant_per_token(x.data_ptr(), x.stride(0), M, K, dtype_code(x), q.data_ptr(),
                               q.stride(0), s.data_ptr(), _stream(x))
    _lib.check(rc, "ll_quant_per_token")
    return q, s


def quant_static(x, scale, q=None, s=None):
    """(int8 [M, K], fp32 scale [M] all equal to *scale): static per-tensor
    quantisation with a calibrated input scale (device fp32 tensor, one element)."""
    _dev(x, scale, q, s)
    M, K = x.shape
    assert x.stride(1) == 1 and scale.dtype == torch.float32 and scale.numel() == 1
    if q is None:
        q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if s is None:
        s = torch.empty((M,), dtype=torch.float32, device=x.device)
    rc = _L.ll_quant_static(x.data_ptr(), x.stride(0), M, K, dtype_code(x), scale.data_ptr(),
                            q.data_ptr(), q.stride(0), s.data_ptr(), _stream(x))
    _lib.check(rc, "ll_quant_static")
    return q, s


class PackedI8Weight:
    """int8 weight [N, K] in the packed streaming layout, with its per-channel scale."""

    def __init__(self, wq, scale):
        _dev(wq, scale)
        N, K = wq.shape
        assert wq.dtype == torch.int8 and wq.stride(1) == 1 and scale.shape == (N,)
        nbytes = _L.ll_gemm_i8_packed_bytes(N, K)
        if nbytes <= 0:
            raise _lib.LiteLangError(f"ll_gemm_i8_pack: K={K} is not a multiple of 256")
        self.shape, self.scale, self.device = (N, K), scale, wq.device
        self.data = torch.empty(nbytes, dtype=torch.uint8, device=wq.device)
        rc = _L.ll_gemm_i8_pack(wq.data_ptr(), wq.stride(0), N, K, self.data.data_ptr(), nbytes,
                                _stream(wq))
        _lib.check(rc, "ll_gemm_i8_pack")


class PackedI8GateUp:
    """int8 [gate; up] weight [2I, K] packed for the fused gate/up + SiLU GEMM."""

    def __init__(self, wq, scale):
        _dev(wq, scale)
        N2, K = wq.shape
        assert wq.dtype == torch.int8 and wq.stride(1) == 1 and N2 % 2 == 0 and scale.shape == (N2,)
        I = N2 // 2
        nbytes = _L.ll_gemm_i8_packed_gate_up_bytes(I, K)
        if nbytes <= 0:
            raise _lib.LiteLangError(f"ll_gemm_i8_pack_gate_up: K={K} is not a multiple of 256")
        self.shape, self.inter, self.scale, self.device = (N2, K), I, scale, wq.device
        self.data = torch.empty(nbytes, dtype=torch.uint8, device=wq.device)
        rc = _L.ll_gemm_i8_pack_gate_up(wq.data_ptr(), wq.stride(0), I, K, self.data.data_ptr(),
                                        nbytes, _stream(wq))
        _lib.check(rc, "ll_gemm_i8_pack_gate_up")


def gemm_i8_gate_up_silu(xq, st, pg: PackedI8GateUp, out):
    """out[M, I] = dtype(u * dtype(silu(g))) of the dequantised int8 gate/up
    product (one launch)."""
    _dev(xq, st, out)
    M, K = xq.shape
    rc = _L.ll_gemm_i8_gate_up_silu_packed(
        xq.data_ptr(), xq.stride(0), pg.data.data_ptr(), M, pg.inter, K, st.data_ptr(),
        pg.scale.data_ptr(), dtype_code(pg.scale), out.data_ptr(), out.stride(0),
        dtype_code(out), _stream(out))
    _lib.check(rc, "ll_gemm_i8_gate_up_silu_packed")
    return out


def gemm_i8_splitk_count(M, N, K) -> int:
    return _L.ll_gemm_i8_splitk_count(M, N, K)


def gemm_i8_splitk_packed(xq, wp: PackedI8Weight, part):
    """int32 partial sums of xq[M, K] @ wq[N, K]^T into part (flat int32); returns splits."""
    _dev(xq, part)
    M, K = xq.shape
    N = wp.shape[0]
    assert wp.shape[1] == K and xq.dtype == torch.int8 and part.dtype == torch.int32
    s = _L.ll_gemm_i8_splitk_count(M, N, K)
    rc = _L.ll_gemm_i8_splitk_packed(xq.data_ptr(), xq.stride(0), wp.data.data_ptr(), M, N, K,
                                     part.data_ptr(), part.numel() * 4, _stream(xq))
    _lib.check(rc, "ll_gemm_i8_splitk_packed")
    return s


def dequant_splitk(part, splits, s_tok, s_ch, out, M, N):
    """out[M, N] fp32 = fp32(sum of int32 partials) * s_tok[m] * fp32(s_ch[n])."""
    _dev(part, s_tok, s_ch, out)
    assert part.dtype == torch.int32 and s_tok.dtype == torch.float32 and out.dtype == torch.float32
    rc = _L.ll_dequant_splitk(part.data_ptr(), splits, s_tok.data_ptr(), s_ch.data_ptr(),
                              dtype_code(s_ch), out.data_ptr(), M, N, _stream(part))
    _lib.check(rc, "ll_dequant_splitk")
    return out


class QuantWeight:
    """W8A8 projection weight: int8 [N, K] with per-channel scales (the model
    dtype when quantised here, the checkpoint's dtype when loaded), its packed
    streaming image when K % 256 == 0, and optionally a calibrated static
    input scale (fp32 device tensor, one element; None = dynamic per token).
    A [gate; up] weight also keeps the 64-row interleaved int8 copy the fused
    prefill gate/up + SiLU tile kernel reads (q_il; None where the layout
    does not apply)."""

    def __init__(self, w=None, gate_up=False):
        self.input_scale = None
        self.packed = self.packed_gu = self.q_il = None
        if w is None:
            return
        self.q, self.scale = quant_weight_per_channel(w)
        self.shape = tuple(w.shape)
        self._pack(gate_up)

    def _pack(self, gate_up):
        """Streaming image for M <= 64: the plain layout, or for a [gate; up]
        weight the fused gate/up + SiLU layout (decode uses only that one),
        plus the interleaved copy for the tile kernel (M > 64)."""
        if gate_up and self.shape[1] % 64 == 0:
            self.q_il = interleave_gate_up(self.q)
        if self.shape[1] % 256 != 0:
            return
        if gate_up:
            self.packed_gu = PackedI8GateUp(self.q, self.scale)
        else:
            self.packed = PackedI8Weight(self.q, self.scale)

    @classmethod
    def from_int8(cls, q, scale, input_scale=None, gate_up=False):
        """Wrap an already quantised weight (a converted checkpoint's int8
        `weight` and `weight_scale`, and its `quant_scale` when present)."""
        _dev(q, scale)
        self = cls()
        N, K = q.shape
        assert q.dtype == torch.int8 and scale.numel() == N
        self.q, self.scale = q.contiguous(), scale.reshape(N).contiguous()
        self.shape = (N, K)
        self._pack(gate_up)
        if input_scale is not None:
            s = float(input_scale)
            if not s > 0.0:
                raise _lib.LiteLangError(f"static input scale must be > 0 (got {s})")
            self.input_scale = torch.tensor([s], dtype=torch.float32, device=q.device)
        return self


class I8Partials:
    """int32 split-K partials [splits, M, N] of an int8 projection with the
    scales that dequantise them (s_tok [M] fp32, s_ch [N])."""

    def __init__(self, part, splits, s_tok, s_ch):
        self.part, self.splits, self.s_tok, self.s_ch = part, splits, s_tok, s_ch


def quant_input(x, qw: QuantWeight):
    """int8 codes and scales of a projection's input: static when the weight
    carries a calibrated input scale, per token otherwise."""
    return quant_per_token(x) if qw.input_scale is None else quant_static(x, qw.input_scale)


def gemm_w8a8_i32(xq, st, qw: QuantWeight) -> I8Partials:
    """The exact int32 product int8(x) @ int8(W)^T (the streaming kernel for
    M <= 64, the int8 tile kernel above that) as partials with their scales."""
    M, K = xq.shape
    N = qw.shape[0]
    if M <= 64 and qw.packed is not None:
        s = gemm_i8_splitk_count(M, N, K)
        part = workspace(xq.device, "w8a8_part", s * M * N * 4).view(torch.int32)
        gemm_i8_splitk_packed(xq, qw.packed, part)
    else:
        s = 1
        part = gemm_i8_i32(xq, qw.q)
    return I8Partials(part, s, st, qw.scale)


def linear_w8a8_fp32(x, qw: QuantWeight, out=None):
    """fp32 [M, N] = dequant(int8(x) @ int8(W)^T): the exact int32 product
    scaled by the activation (per-token, or the static input scale) and
    per-channel weight scales."""
    _dev(x, out)
    M = x.shape[0]
    N = qw.shape[0]
    xq, st = quant_input(x, qw)
    p = gemm_w8a8_i32(xq, st, qw)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    return dequant_splitk(p.part, p.splits, p.s_tok, p.s_ch, out, M, N)


def add_rmsnorm_splitk_i32(h, p: I8Partials, gamma, eps, out=None, quant=False):
    """add_rmsnorm_splitk from int32 partials (dequantised inline); with quant,
    also returns the output's per-token int8 codes and scales."""
    _dev(h, p.part, gamma, out)
    M, N = h.shape
    if out is None:
        out = torch.empty_like(h)
    q = torch.empty((M, N), dtype=torch.int8, device=h.device) if quant else None
    s = torch.empty((M,), dtype=torch.float32, device=h.device) if quant else None
    rc = _L.ll_add_rmsnorm_splitk_i32(
        h.data_ptr(), h.stride(0), p.part.data_ptr(), p.splits, p.s_tok.data_ptr(),
        p.s_ch.data_ptr(), dtype_code(p.s_ch), gamma.data_ptr(), out.data_ptr(), out.stride(0), M,
        N, float(eps), dtype_code(h), q.data_ptr() if quant else None, N,
        s.data_ptr() if quant else None, _stream(h))
    _lib.check(rc, "ll_add_rmsnorm_splitk_i32")
    return (out, q, s) if quant else out


def silu_and_mul_splitk_i32(p: I8Partials, out):
    """silu_and_mul_splitk from int32 partials of the [M, 2N] product."""
    _dev(p.part, out)
    M, N = out.shape
    rc = _L.ll_silu_and_mul_splitk_i32(p.part.data_ptr(), p.splits, p.s_tok.data_ptr(),
                                       p.s_ch.data_ptr(), dtype_code(p.s_ch), out.data_ptr(),
                                       out.stride(0), M, N, dtype_code(out), _stream(out))
    _lib.check(rc, "ll_silu_and_mul_splitk_i32")
    return out


def linear_w8a8(x, qw: QuantWeight, bias=None):
    """dtype(linear_w8a8_fp32(x) + bias), the rounding of the fused consumers
    (above 64 rows in one launch: the tile kernel's dequantising epilogue
    evaluates the same fp32 expression)."""
    M, K = x.shape
    N = qw.shape[0]
    if (M > 64 and x.dtype in (torch.bfloat16, torch.float16) and gemm_i8_tiled_supported(M, N, K)
            and (bias is None or bias.dtype == x.dtype)):
        xq, st = quant_input(x, qw)
        return gemm_i8_tiled(xq, st, qw.q, qw.scale, bias, out_dtype=x.dtype)
    y = linear_w8a8_fp32(x, qw)
    if bias is not None:
        y = y + bias.float()
    return y.to(x.dtype)
