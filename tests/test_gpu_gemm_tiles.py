"""The prefill tile GEMMs (gemm_tiles.hip) against the CPU oracle.

* bf16 / fp16 products (with and without bias, ragged M and N edges, strided
  activation rows) within 2e-2 + one bf16 ulp of |y| of the float64 product
  of the same rounded operands;
* the fused gate/up + SiLU_and_Mul epilogue equals the unfused sequence (the
  tile GEMM, then ll_silu_and_mul) bit for bit, and the oracle's
  silu_and_mul within the same bar;
* int8: the int32 sums equal the oracle's exact integer product bit for bit
  (ragged edges, K up to 11008); the dequantising epilogue equals
  fp32(acc) * s_tok * fp32(s_ch) (+ bias, rounded) computed on the host from
  those exact sums, bit for bit; the int8 gate/up + SiLU epilogue equals the
  dequantised product followed by silu_and_mul bit for bit.
"""
import pytest
import torch

from oracle import ops as O

pytestmark = pytest.mark.gpu

BF16_ATOL, BF16_RTOL = 2e-2, 2.0 ** -7


def _ops():
    from lite_lang_amd import ops
    return ops


def _close(y, ref):
    excess = (y.detach().cpu().double() - ref.double()).abs() - (BF16_ATOL + BF16_RTOL * ref.double().abs())
    return float(excess.max())


@pytest.mark.parametrize("M,N,K,dtype,bias", [
    (300, 256, 64, torch.bfloat16, True), (257, 260, 96, torch.bfloat16, False),
    (1000, 2560, 2048, torch.bfloat16, True), (4097, 2048, 11008, torch.bfloat16, False),
    (513, 2048, 2048, torch.float16, True), (65, 1536, 8960, torch.bfloat16, False)])
def test_gemm_tiled_matches_oracle(cuda, M, N, K, dtype, bias):
    g = torch.Generator().manual_seed(81)
    x = torch.randn(M, K + 32, generator=g).to(dtype)[:, :K]  # strided rows
    w = (torch.randn(N, K, generator=g) * 0.05).to(dtype)
    b = torch.randn(N, generator=g).to(dtype) if bias else None
    print(f"case: gemm_tiled M={M} N={N} K={K} {dtype} bias={bias}", flush=True)
    y = _ops().gemm_tiled(x.to(cuda), w.to(cuda), b.to(cuda) if bias else None)
    ref = O.linear(x, w, b)
    assert _close(y, ref) <= 0


def test_ll_gemm_routes_prefill_to_tiles(cuda):
    """ll_gemm (the generic entry) above 64 rows gives the tile kernel's result."""
    g = torch.Generator().manual_seed(82)
    x = torch.randn(200, 512, generator=g).bfloat16().to(cuda)
    w = (torch.randn(768, 512, generator=g) * 0.05).bfloat16().to(cuda)
    ops = _ops()
    print("case: ll_gemm routing", flush=True)
    assert torch.equal(ops.gemm(x, w), ops.gemm_tiled(x, w))


@pytest.mark.parametrize("M,I,K", [(300, 256, 256), (1000, 11008, 2048), (77, 8960, 1536)])
def test_gate_up_silu_tiled_equals_unfused(cuda, M, I, K):
    g = torch.Generator().manual_seed(83)
    x = torch.randn(M, K, generator=g).bfloat16()
    wgu = (torch.randn(2 * I, K, generator=g) * (1.25 / K ** 0.5)).bfloat16()
    ops = _ops()
    print(f"case: gate_up_silu_tiled M={M} I={I} K={K}", flush=True)
    xd, wd = x.to(cuda), wgu.to(cuda)
    wil = ops.interleave_gate_up(wd)
    got = ops.gate_up_silu_tiled(xd, wil)
    gu = ops.gemm_tiled(xd, wd)
    want = ops.silu_and_mul(gu, out=torch.empty((M, I), dtype=gu.dtype, device=cuda))
    assert torch.equal(got, want)
    ref = O.silu_and_mul(O.rnd(O.linear(x, wgu), torch.bfloat16), torch.bfloat16)
    assert _close(got, ref) <= 0


@pytest.mark.parametrize("M,N,K", [(300, 256, 64), (259, 2560, 2048), (1000, 2048, 11008),
                                   (4100, 22016, 256)])
def test_gemm_i8_tiled_exact(cuda, M, N, K):
    g = torch.Generator().manual_seed(84)
    xq = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    wq = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    print(f"case: gemm_i8_i32_tiled M={M} N={N} K={K}", flush=True)
    got = _ops().gemm_i8_i32_tiled(xq.to(cuda), wq.to(cuda)).cpu()
    assert torch.equal(got, O.int8_gemm_i32(xq, wq))


@pytest.mark.parametrize("out_dtype,sdt,bias", [(torch.bfloat16, torch.bfloat16, True),
                                                (torch.float16, torch.float16, False),
                                                (torch.float32, torch.float32, False)])
def test_gemm_i8_tiled_dequant_bit_exact(cuda, out_dtype, sdt, bias):
    g = torch.Generator().manual_seed(85)
    M, N, K = 517, 1024, 2048
    xq = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    wq = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    st = torch.rand(M, generator=g) * 0.01 + 1e-4
    sc = (torch.rand(N, generator=g) * 0.01 + 1e-4).to(sdt)
    b = torch.randn(N, generator=g).to(out_dtype) if bias else None
    print(f"case: gemm_i8_tiled dequant {out_dtype} scales {sdt} bias={bias}", flush=True)
    got = _ops().gemm_i8_tiled(xq.to(cuda), st.to(cuda), wq.to(cuda), sc.to(cuda),
                               b.to(cuda) if bias else None, out_dtype=out_dtype).cpu()
    v = O.dequant_int32(O.int8_gemm_i32(xq, wq), st, sc)  # fp32, the kernel's order
    if bias:
        v = v + b.float()
    assert torch.equal(got, v.to(out_dtype))


def test_gemm_i8_gate_up_silu_tiled_bit_exact(cuda):
    g = torch.Generator().manual_seed(86)
    M, I, K = 300, 1024, 1024
    xq = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    wq = torch.randint(-128, 128, (2 * I, K), generator=g, dtype=torch.int8)
    st = torch.rand(M, generator=g) * 0.001 + 1e-5
    sc = (torch.rand(2 * I, generator=g) * 0.001 + 1e-5).bfloat16()
    ops = _ops()
    print("case: gemm_i8_gate_up_silu_tiled", flush=True)
    xd, wd, std, scd = xq.to(cuda), wq.to(cuda), st.to(cuda), sc.to(cuda)
    got = ops.gemm_i8_gate_up_silu_tiled(xd, std, ops.interleave_gate_up(wd), scd)
    gu = ops.gemm_i8_tiled(xd, std, wd, scd, out_dtype=torch.bfloat16)
    want = ops.silu_and_mul(gu, out=torch.empty((M, I), dtype=torch.bfloat16, device=cuda))
    assert torch.equal(got, want)


@pytest.mark.parametrize("M,N,K,pad", [(70, 100, 36, 0), (300, 50, 100, 3), (129, 256, 128, 0),
                                       (65, 2048, 8960, 0), (262200, 8, 36, 0)])
def test_gemm_i8_i32_any_shape_exact(cuda, M, N, K, pad):
    """ll_gemm_i8_i32 (the W8A8 prefill product): the tile kernel where its
    layout holds, the plain dot-product kernel elsewhere (K % 64 != 0, odd
    row strides; more than 65535 x 4 rows in several launches); exact int32
    sums either way."""
    g = torch.Generator().manual_seed(87)
    xfull = torch.randint(-128, 128, (M, K + pad), generator=g, dtype=torch.int8)
    wq = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    print(f"case: gemm_i8_i32 M={M} N={N} K={K} pad={pad}", flush=True)
    got = _ops().gemm_i8_i32(xfull.to(cuda)[:, :K], wq.to(cuda)).cpu()  # row stride K + pad
    assert torch.equal(got, O.int8_gemm_i32(xfull[:, :K].contiguous(), wq))


def test_gemm_tiled_rows_past_4gib_chunked_bit_exact(cuda):
    """Activations spanning more than 4 GiB are launched in row chunks (the
    kernel's source offsets are 32-bit): the rows around the first chunk
    boundary equal the same kernel's result on those rows alone (a
    size-independent property; the oracle would take minutes at this size)."""
    K, N = 2048, 256
    row_b = K * 2
    chunk = ((((1 << 32) - 128) // row_b) // 256) * 256  # rows per launch, as the host computes
    M = chunk + 1024
    ops = _ops()
    g = torch.Generator(device=cuda).manual_seed(88)
    print(f"case: gemm_tiled M={M} (chunk {chunk}) N={N} K={K}", flush=True)
    x = torch.randn(M, K, device=cuda, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, device=cuda, generator=g) * 0.05).to(torch.bfloat16)
    y = ops.gemm_tiled(x, w)
    lo, hi = chunk - 512, chunk + 512
    ref = ops.gemm_tiled(x[lo:hi].contiguous(), w)
    assert torch.equal(y[lo:hi], ref)
    assert torch.equal(y[-300:], ops.gemm_tiled(x[-300:].contiguous(), w))
    del x, y
    torch.cuda.empty_cache()
