// Dense projections Y[M, N] = X[M, K] . W[N, K]^T (+ bias), gfx950.
//
// Replaces the cuBLAS products of the reference token loop
// (litelang/models/qwen2/layer/transformer_layer.py:80,82,95-109,193 and
// post_layer.py:20-22). W keeps the nn.Linear [out, in] layout so that both
// MFMA operands are 16-byte k-contiguous loads.
//
// Kernels:
//   * M <= 64 (the decode step) is weight streaming: two kernels (LDS-staged
//     for wide/deep weights, direct for the small projections, below), MFMA
//     v_mfma_f32_16x16x32 with the tokens as the 16-wide N side. Narrow N is
//     split over K across workgroups into fp32 partials, which either a
//     reduce kernel (ll_gemm) or the consumer kernel of the model
//     (ll_gemm_splitk + the *_splitk entry points) sums in a fixed order;
//   * tiled (M > 64, prefill): 128x128x64 LDS tiles, 2x2 waves of 64x64,
//     register-staged prefetch of the next k tile;
//   * fp32: plain FMA tiles for the fp32 parity path.
#include "ll_common.h"

#include <type_traits>

namespace {

// 16-byte operand fragment of one lane and the MFMA accumulator, per element type
template <typename T> struct Vec8;
template <> struct Vec8<__bf16> { typedef bf16x8 type; };
template <> struct Vec8<_Float16> { typedef f16x8 type; };
template <> struct Vec8<int8_t> { typedef i32x4 type; };  // 16 int8
template <typename T> struct AccOf { typedef f32x4 type; };
template <> struct AccOf<int8_t> { typedef i32x4 type; };

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// int8: one 16-byte fragment per lane is a 64-deep k step (exact int32 sums)
__device__ __forceinline__ i32x4 mfma16x16x32(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

template <typename V8> __device__ __forceinline__ V8 zero8() {
  V8 z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = 0;
  return z;
}

// ---------------------------------------------------------------- skinny
// Output of the M <= 64 kernels: if `part` is non-null, fp32 partial sums
// part[split][m][n] (N contiguous, no bias); else Y[m][n] = T(sum + bias[n]).

// Wait until at most N of this wave's vector memory operations are in flight.
template <int N_> __device__ __forceinline__ void vm_wait() {
  static_assert(N_ >= 0 && N_ < 64, "vmcnt is a 6-bit counter");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
}

// Workgroup barrier that waits for nothing but this wave's LDS reads. The
// caller has already waited (vm_wait) for its own LDS DMA of the stage the
// other waves will read. __syncthreads() would also drain every outstanding
// global load, including the DMA of the stage being prefetched, and so
// serialise the pipeline.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16 B global -> LDS DMA of one lane (lane i of the wave lands at lds + 16 i).
// Kept out of the kernel templates: a dependent call of this device-only
// builtin makes the host pass drop the template's launch stub.
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}
// Same, marked non-temporal: used for the weight stream, read once, so that it
// does not evict the small, reused activation tensor from L2.
__device__ __forceinline__ void dma16_stream(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 2 /* nt */);
}

// (1) Wide N: weight rows streamed through LDS. A workgroup (4 waves) owns 64
// rows; every stage DMA's (global_load_lds_dwordx4, no VGPR staging) a
// 64-row x 128-k weight tile and the matching 16*MB-row activation tile into
// LDS, with 256 contiguous bytes per row per wave instruction. The 16 B chunk
// index of every row is XOR-swizzled by (row & 15) so the MFMA operand reads
// (16 rows x 16 B per 16 lanes) are bank-conflict free. NST stage buffers
// form a ring: while stage st is multiplied, stages st+1 .. st+NST-1 are in
// flight. One barrier per stage: after it, every wave has finished stage
// st-1, so its buffer is refilled with stage st+NST-1.
constexpr int kDmaKC = 128, kDmaTR = 64;

// Wait for the oldest in-flight stage when `later` younger stages of C
// operations each may stay in flight (later <= NST - 2).
template <int C, int NST>
__device__ __forceinline__ void wait_stage(int later) {
  if constexpr (NST >= 4) {
    if (later >= 2) { vm_wait<2 * C>(); return; }
  }
  if constexpr (NST >= 3) {
    if (later >= 1) { vm_wait<C>(); return; }
  }
  vm_wait<0>();
}

// PK: W is the pre-packed layout of ll_gemm_pack (every stage of every row
// tile one contiguous, already swizzled 16 KB block, blocks ordered chunk-
// major), so concurrent workgroups stream neighbouring blocks.
// EPI 1 (with PK and the gate/up tile layout of ll_gemm_pack_gate_up, one
// split): tile rows 0..TR/2-1 are gate channels (TR/2)t.., the other TR/2 rows
// the matching up channels; the epilogue writes Y[m, c] =
// T(T(up) * T(silu(T(gate)))) for the TR/2 channels of the tile (N = 2 *
// channels), the rounding sequence of ll_silu_and_mul_splitk applied to the
// same fp32 sums.
// EPI 2 (one split, bf16/fp16 operands, no partials): Y as EPI 0, and for
// every token the tile's largest Y value with its first channel index,
// written to e8.am_val / e8.am_idx[token][tile] (the first pass of a
// first-index argmax over the row; argmax_final_kernel finishes it).
// int8 gate/up epilogue (EPI 1 with int8 operands): the int32 sums are
// dequantised as fp32(acc) * s_tok[m] * fp32(s_ch[col]) (col = channel for
// gate, I + channel for up) and SiLU_and_Mul is written to y (type TO).
struct I8Epi {
  const float* s_tok;
  const void* s_ch;
  int s_ch_dtype;
  void* y;
  int64_t ldy;
  // EPI 2: per-token argmax partials of the tile, [M][tiles] (value, index)
  float* am_val;
  int* am_idx;
};

template <typename T, int MB, int NST, bool PK, int EPI = 0, int TR = 64, typename TO = T>
__global__ __launch_bounds__(256) void gemm_dma_kernel(const T* __restrict__ X, int64_t ldx,
                                                       const T* __restrict__ W, int64_t ldw,
                                                       int M, int N, int K, int ksps, int rotate,
                                                       const T* __restrict__ bias,
                                                       T* __restrict__ Y, int64_t ldy,
                                                       float* __restrict__ part, I8Epi e8) {
  // (what the first stage's copies need leads the list: gfx950 preloads the
  // leading 16 SGPRs of scalar arguments at dispatch, so those copies do not
  // wait for the load of the rest)
  static_assert(NST >= 2 && NST <= 4, "2 to 4 stage buffers");
  typedef typename Vec8<T>::type V8;
  typedef typename AccOf<T>::type AccT;
  constexpr int ES = (int)sizeof(T);
  static_assert(TR == 64 || TR == 96 || TR == 128, "64-, 96- or 128-row tiles");
  constexpr int XR = 16 * MB;
  constexpr int RB = (TR / 16 + 3) / 4;   // 16-row MFMA blocks per wave (at most)
  constexpr int KC = 256 / ES;            // elements per 256-byte row chunk (one stage)
  constexpr int CE = 16 / ES;             // elements per 16-byte fragment
  constexpr int KSTEP = 4 * CE;           // k per MFMA: 32 (16-bit types), 64 (int8)
  constexpr int ROWB = 256, CH = ROWB / 16, RPI = 64 / CH;  // 16 chunks, 4 rows/instr
  constexpr int W_PER_WAVE = (TR / RPI) / 4;
  constexpr int X_PER_WAVE = (XR / RPI) / 4;
  constexpr int C = W_PER_WAVE + X_PER_WAVE;  // DMA instructions per wave per stage
  constexpr int STAGE_B = (TR + XR) * ROWB;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, j = lane >> 4;
  const int row0 = blockIdx.x * TR;
  const int split = blockIdx.y;
  // the tile's 16-row MFMA blocks per wave: RB consecutive ones with 64 and
  // 128 rows; with 96 rows waves 0 and 1 take blocks w and w + 4, waves 2
  // and 3 block w alone (nb: the wave's block count, a scalar)
  auto blk = [&](int b) { return TR == 96 ? wave + 4 * b : wave * RB + b; };
  const int nb = TR == 96 ? (wave < 2 ? 2 : 1) : RB;
  const int k_beg = split * ksps * KSTEP;
  const int k_end = min(K, k_beg + ksps * KSTEP);
  const int nst = (k_end - k_beg) / KC;
  const int lr_in = lane / CH, p = lane % CH;
  // optional per-workgroup rotation of the k-chunk order, so that concurrent
  // workgroups read different column ranges of their rows
  const int rot = (rotate && nst > 0) ? (int)(blockIdx.x % nst) : 0;
  auto issue = [&](int st) {
    char* base = smem + (st % NST) * STAGE_B;
    int kc = st + rot;
    if (kc >= nst) kc -= nst;
    const int k0 = k_beg + kc * KC;
#pragma unroll
    for (int q = 0; q < W_PER_WAVE; ++q) {
      const int ii = wave * W_PER_WAVE + q;
      if constexpr (PK) {
        const char* g = (const char*)W + ((int64_t)(k0 / KC) * gridDim.x + blockIdx.x) * (TR * ROWB) +
                        ii * 1024 + lane * 16;
        dma16_stream(g, base + ii * 1024);
      } else {
        const int r = ii * RPI + lr_in;
        const T* g = W + (int64_t)min(row0 + r, N - 1) * ldw + k0 + (p ^ (r & 15)) * CE;
        dma16_stream(g, base + ii * 1024);
      }
    }
#pragma unroll
    for (int q = 0; q < X_PER_WAVE; ++q) {
      const int ii = wave + q * 4;
      const int r = ii * RPI + lr_in;
      const T* g = X + (int64_t)min(r, M - 1) * ldx + k0 + (p ^ (r & 15)) * CE;
      dma16(g, base + TR * ROWB + ii * 1024);
    }
  };
  AccT acc[RB][MB];
#pragma unroll
  for (int b = 0; b < RB; ++b)
#pragma unroll
    for (int t = 0; t < MB; ++t) acc[b][t] = (AccT){0, 0, 0, 0};
  // int8 gate/up epilogue scales, loaded (clamped, unconditionally) before the
  // weight stream so that their latency hides behind it: the token scales of
  // this lane's tokens and the raw bits of the channel scales of its gate
  // (waves 0, 1) or up (waves 2, 3) channels, converted only in the epilogue
  // (a conversion here would wait for the loads before the stream starts)
  float e_st[MB];
  uint32_t e_sc[RB][4];
  if constexpr (ES == 1 && EPI == 1) {
    const int I = N / 2;
#pragma unroll
    for (int t = 0; t < MB; ++t) e_st[t] = e8.s_tok[min(16 * t + n, M - 1)];
    auto load_sc = [&](auto tag) {
      typedef decltype(tag) S;
      const S* s = (const S*)e8.s_ch;
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int row = 16 * blk(min(b, nb - 1)) + 4 * j;  // tile row of acc[b][.][0]
        const bool up = row >= TR / 2;
        const int cbase = blockIdx.x * (TR / 2) + row - (up ? TR / 2 : 0);
        const int coff = up ? I : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) e_sc[b][i] = s[coff + min(cbase + i, I - 1)];
      }
    };
    if (e8.s_ch_dtype == LL_F32) load_sc(uint32_t{});
    else load_sc((unsigned short){});
  }
#pragma unroll
  for (int st = 0; st < NST - 1; ++st)
    if (st < nst) issue(st);
  for (int st = 0; st < nst; ++st) {
    // issued so far: stages 0 .. min(nst, st + NST - 1) - 1
    wait_stage<C, NST>(min(NST - 2, nst - 1 - st));
    lds_barrier();
    if (st + NST - 1 < nst) issue(st + NST - 1);  // into the buffer of stage st-1
    const char* wb = smem + (st % NST) * STAGE_B;
    const char* xb = wb + TR * ROWB;
#pragma unroll
    for (int s = 0; s < KC / KSTEP; ++s) {
      V8 a[RB];
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        if (b < nb) {
          const int lr = 16 * blk(b) + n;
          a[b] = *(const V8*)(wb + lr * ROWB + (((4 * s + j) ^ (lr & 15)) * 16));
        }
      }
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        const int xr = 16 * t + n;
        const V8 xv = *(const V8*)(xb + xr * ROWB + (((4 * s + j) ^ (xr & 15)) * 16));
#pragma unroll
        for (int b = 0; b < RB; ++b)
          if (b < nb) acc[b][t] = mfma16x16x32(a[b], xv, acc[b][t]);
      }
    }
  }
  // acc[b][t][i] = Y[token 16t + n][channel row0 + 16*blk(b) + 4j + i], b < nb
  if constexpr (EPI == 1) {
    // gate/up, one split: every wave puts its sums (int8: dequantised as
    // fp32(acc) * s_tok[m] * fp32(s_ch[col])) into LDS rows [token][channel],
    // gate from waves 0, 1 and up from waves 2, 3; then each thread takes 4
    // consecutive channels of one token through SiLU_and_Mul with the rounding
    // sequence of silu_and_mul_splitk, computed before its one guarded 8-byte
    // store. All four waves share the arithmetic.
    constexpr int HALF = TR / 2;      // gate (and up) channels of the tile
    constexpr int PITCH = HALF + 4;   // floats per LDS row: rows shift by 16 B across the banks
    constexpr int XT = 16 * MB;       // token rows
    const int I = N / 2;
    float* gbuf = (float*)smem;
    float* ubuf = gbuf + XT * PITCH;
    float vs[RB][MB][4];
    if constexpr (ES == 1) {
      float sc[RB][4];
      auto cvt = [&](auto dt) {
#pragma unroll
        for (int b = 0; b < RB; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[b][i] = ll_scale_bits_to_f32(e_sc[b][i], decltype(dt)::value);
      };
      if (e8.s_ch_dtype == LL_F16) cvt(std::integral_constant<int, LL_F16>{});
      else if (e8.s_ch_dtype == LL_BF16) cvt(std::integral_constant<int, LL_BF16>{});
      else cvt(std::integral_constant<int, LL_F32>{});
#pragma unroll
      for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int t = 0; t < MB; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) vs[b][t][i] = (float)acc[b][t][i] * e_st[t] * sc[b][i];
    } else {
#pragma unroll
      for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int t = 0; t < MB; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) vs[b][t][i] = acc[b][t][i];
    }
    lds_barrier();  // every wave is done reading the last stage
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      if (b < nb) {
        // a 16-row block is all gate (tile rows < HALF) or all up channels
        const int row = 16 * blk(b) + 4 * j;
        const bool up = row >= HALF;
        float* dst = up ? ubuf : gbuf;
        const int cl = row - (up ? HALF : 0);
#pragma unroll
        for (int t = 0; t < MB; ++t)
          *(f32x4*)(dst + (16 * t + n) * PITCH + cl) =
              (f32x4){vs[b][t][0], vs[b][t][1], vs[b][t][2], vs[b][t][3]};
      }
    }
    lds_barrier();
    TO* Yo = ES == 1 ? (TO*)e8.y : (TO*)Y;
    const int64_t ly = ES == 1 ? e8.ldy : ldy;
    const bool vec = ((I | ly) & 3) == 0;
    constexpr int QPR = HALF / 4;     // channel quads per token row
    constexpr int QUADS = XT * QPR;
#pragma unroll
    for (int r = 0; r < (QUADS + 255) / 256; ++r) {
      const int q = r * 256 + (int)threadIdx.x;
      if (QUADS % 256 != 0 && q >= QUADS) break;
      const int tok = q / QPR, cq = (q - tok * QPR) * 4;
      const f32x4 g4 = *(const f32x4*)(gbuf + tok * PITCH + cq);
      const f32x4 u4 = *(const f32x4*)(ubuf + tok * PITCH + cq);
      TO y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float g = ll_to_f32(ll_from_f32<TO>(g4[e]));
        const float u = ll_to_f32(ll_from_f32<TO>(u4[e]));
        const TO sv = ll_from_f32<TO>(ll_silu_f32(g));
        y[e] = ll_from_f32<TO>(u * ll_to_f32(sv));
      }
      const int c0 = blockIdx.x * HALF + cq;
      if (tok < M && c0 < I) {
        TO* yp = Yo + (int64_t)tok * ly + c0;
        if (vec) {
          typedef TO V4 __attribute__((ext_vector_type(4)));
          *(V4*)yp = (V4){y[0], y[1], y[2], y[3]};
        } else {
          for (int e = 0; e < 4 && c0 + e < I; ++e) yp[e] = y[e];
        }
      }
    }
    return;
  } else if constexpr (EPI == 2) {
    // fp32 logits and the argmax's first pass: every lane stores its RB
    // channel quads of each token and keeps its (value, first index) per
    // token, then the 4 lane groups of a token (shuffles) and the 4 waves
    // (LDS, free after the last stage) merge theirs into the tile's partial.
    // The picks are selects, not branches: no exec-masked joins.
    static_assert(std::is_same<TO, float>::value, "the argmax epilogue writes fp32 logits");
    float* Yf = (float*)(void*)Y;
    const bool vec = ((ldy & 3) == 0) && (((uintptr_t)Yf & 15) == 0);
    float bv[MB];
    int bi[MB];
#pragma unroll
    for (int t = 0; t < MB; ++t) { bv[t] = -INFINITY; bi[t] = 0x7fffffff; }
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      if (b >= nb) continue;
      const int ch = row0 + 16 * blk(b) + 4 * j;
      float bb[4] = {0.f, 0.f, 0.f, 0.f};
      if (bias != nullptr) {
#pragma unroll
        for (int i = 0; i < 4; ++i) bb[i] = ll_to_f32(bias[min(ch + i, N - 1)]);
      }
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        const int tok = 16 * t + n;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = acc[b][t][i] + bb[i];
          // channel indices rise with i, so a tie keeps the earlier pick
          const bool take = (ch + i < N) & ((v[i] > bv[t]) | ((v[i] == bv[t]) & (bi[t] == 0x7fffffff)));
          bv[t] = take ? v[i] : bv[t];
          bi[t] = take ? ch + i : bi[t];
        }
        if (tok < M && ch < N) {
          float* yp = Yf + (int64_t)tok * ldy + ch;
          if (vec && ch + 3 < N) {
            *(f32x4*)yp = (f32x4){v[0], v[1], v[2], v[3]};
          } else {
            for (int i = 0; i < 4 && ch + i < N; ++i) yp[i] = v[i];
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < MB; ++t) {
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        const float ov = __shfl_xor(bv[t], o, 64);
        const int oi = __shfl_xor(bi[t], o, 64);
        const bool take = (ov > bv[t]) | ((ov == bv[t]) & (oi < bi[t]));
        bv[t] = take ? ov : bv[t];
        bi[t] = take ? oi : bi[t];
      }
    }
    lds_barrier();  // every wave is done reading the last stage
    float* sval = (float*)smem;
    int* sidx = (int*)(sval + 4 * XR);
    if (j == 0) {
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        sval[wave * XR + 16 * t + n] = bv[t];
        sidx[wave * XR + 16 * t + n] = bi[t];
      }
    }
    lds_barrier();
    const int tok = (int)threadIdx.x;
    if (tok < M) {
      float v = sval[tok];
      int i = sidx[tok];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const float ov = sval[w * XR + tok];
        const int oi = sidx[w * XR + tok];
        const bool take = (ov > v) | ((ov == v) & (oi < i));
        v = take ? ov : v;
        i = take ? oi : i;
      }
      e8.am_val[(int64_t)tok * gridDim.x + blockIdx.x] = v;
      e8.am_idx[(int64_t)tok * gridDim.x + blockIdx.x] = i;
    }
    return;
  } else if constexpr (ES == 1) {
    // int8: exact int32 partial sums, part[split][m][n] (part points at int32)
    int32_t* ip = (int32_t*)part;
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      if (b >= nb) continue;
      const int ch = row0 + 16 * blk(b) + 4 * j;
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        const int tok = 16 * t + n;
        if (tok >= M || ch >= N) continue;
        int32_t* pp = ip + ((int64_t)split * M + tok) * N + ch;
        if (ch + 3 < N && (N & 3) == 0) {
          *(i32x4*)pp = acc[b][t];
        } else {
          for (int i = 0; i < 4 && ch + i < N; ++i) pp[i] = acc[b][t][i];
        }
      }
    }
    return;
  } else {
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      if (b >= nb) continue;
      const int ch = row0 + 16 * blk(b) + 4 * j;
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        const int tok = 16 * t + n;
        if (tok >= M || ch >= N) continue;
        if (part != nullptr) {
          float* pp = part + ((int64_t)split * M + tok) * N + ch;
          if (ch + 3 < N && (N & 3) == 0) {
            *(f32x4*)pp = acc[b][t];
          } else {
            for (int i = 0; i < 4 && ch + i < N; ++i) pp[i] = acc[b][t][i];
          }
        } else {
          // (TO: the output type, T or fp32 -- Y then points at TO elements)
          TO* yp = (TO*)(void*)Y + (int64_t)tok * ldy + ch;
          for (int i = 0; i < 4 && ch + i < N; ++i)
            yp[i] = ll_from_f32<TO>(acc[b][t][i] + (bias != nullptr ? ll_to_f32(bias[ch + i]) : 0.f));
        }
      }
    }
  }
}

// Packed weight layout for the DMA kernel with tr-row tiles (64 or 128):
// block (kc, t) = rows tr*t..tr*t+tr-1, row chunk kc (256 bytes: 128 bf16/fp16
// or 256 int8 columns), stored as the LDS image of that stage (unit
// u = 64 * ii + lane holds row 4 ii + lane / 16, 16 B chunk
// (lane % 16) ^ (row & 15)); blocks ordered kc-major; rows >= N are zero.
// gu_half > 0: W is [gate; up] with gu_half rows each, and tile t takes gate
// rows (tr/2)t.. as its rows 0..tr/2-1 and the same up rows as the rest.
__global__ __launch_bounds__(256) void gemm_pack_kernel(const u32x4* __restrict__ W, int64_t ldw16,
                                                        u32x4* __restrict__ out, int N, int tiles,
                                                        int64_t units, int gu_half, int tr) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const int per_blk = tr * 16;  // 16 B units of one block
  const int64_t blk = u / per_blk;
  const int within = (int)(u - blk * per_blk);
  const int ii = within >> 6, lane = within & 63;
  const int kc = (int)(blk / tiles), t = (int)(blk - (int64_t)kc * tiles);
  const int r = ii * 4 + (lane >> 4);
  const int c = (lane & 15) ^ (r & 15);
  int row = t * tr + r;
  bool ok = row < N;
  if (gu_half > 0) {
    const int half = tr / 2;
    const int ch = t * half + (r % half);
    ok = ch < gu_half;
    row = (r < half) ? ch : gu_half + ch;
  }
  u32x4 v = {0u, 0u, 0u, 0u};
  if (ok) v = W[(int64_t)row * ldw16 + (int64_t)kc * (kDmaKC / 8) + c];
  out[u] = v;
}

// (2) Narrow N: direct operand loads. A workgroup owns 16*WR rows; its KW
// waves interleave over the 32-wide k-steps with U steps per group, loads of
// group g+1 in flight while group g is multiplied (register double buffer).
// Row and token indices are clamped into the tensors (their results are
// discarded), so the steady loop has no divergent branches; a masked tail
// handles K % 32 != 0.
template <typename T, int MB, int WR, int KW, int U>
__global__ __launch_bounds__(64 * KW) void gemm_direct_kernel(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, T* __restrict__ Y, int64_t ldy, float* __restrict__ part, int M,
    int N, int K, int ksps) {
  typedef typename Vec8<T>::type V8;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, j = lane >> 4;
  const int row0 = blockIdx.x * (16 * WR);
  const int split = blockIdx.y;
  const int ksteps = (K + 31) / 32;
  const int full = K / 32;  // k-steps with all 32 columns inside K
  const int kb = split * ksps, ke = min(ksteps, kb + ksps);
  const T* wrow[WR];
#pragma unroll
  for (int r = 0; r < WR; ++r) wrow[r] = W + (int64_t)min(row0 + 16 * r + n, N - 1) * ldw + 8 * j;
  const T* xrow[MB];
#pragma unroll
  for (int t = 0; t < MB; ++t) xrow[t] = X + (int64_t)min(16 * t + n, M - 1) * ldx + 8 * j;
  f32x4 acc[WR][MB];
#pragma unroll
  for (int r = 0; r < WR; ++r)
#pragma unroll
    for (int t = 0; t < MB; ++t) acc[r][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // this wave's k-steps: kb + wave + KW*i, i < per_wave; the first `safe` are full
  const int per_wave = max(0, (ke - kb - wave + KW - 1) / KW);
  const int safe = max(0, min(per_wave, (min(ke, full) - kb - wave + KW - 1) / KW));
  const int groups = safe / U;
  V8 wv[2][U][WR], xv[2][U][MB];
  auto load = [&](int buf, int g) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ks = kb + wave + KW * (g * U + u);
#pragma unroll
      for (int r = 0; r < WR; ++r) wv[buf][u][r] = *(const V8*)(wrow[r] + ks * 32);
#pragma unroll
      for (int t = 0; t < MB; ++t) xv[buf][u][t] = *(const V8*)(xrow[t] + ks * 32);
    }
  };
  auto compute = [&](int buf) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < WR; ++r)
#pragma unroll
        for (int t = 0; t < MB; ++t) acc[r][t] = mfma16x16x32(wv[buf][u][r], xv[buf][u][t], acc[r][t]);
  };
  if (groups > 0) {
    load(0, 0);
    int g = 0;
    for (; g + 1 < groups; g += 2) {
      load(1, g + 1);
      compute(0);
      if (g + 2 < groups) load(0, g + 2);
      compute(1);
    }
    if (g < groups) compute(0);
  }
  for (int i = groups * U; i < per_wave; ++i) {
    const int ks = kb + wave + KW * i;
    const bool kok = ks * 32 + 8 * j < K;
    V8 w1[WR], x1[MB];
#pragma unroll
    for (int r = 0; r < WR; ++r) w1[r] = kok ? *(const V8*)(wrow[r] + ks * 32) : zero8<V8>();
#pragma unroll
    for (int t = 0; t < MB; ++t) x1[t] = kok ? *(const V8*)(xrow[t] + ks * 32) : zero8<V8>();
#pragma unroll
    for (int r = 0; r < WR; ++r)
#pragma unroll
      for (int t = 0; t < MB; ++t) acc[r][t] = mfma16x16x32(w1[r], x1[t], acc[r][t]);
  }
  // acc[r][t][i] = Y[token 16t + n][channel row0 + 16r + 4j + i]; merge the KW waves
  __shared__ float red[KW][WR * 16][MB * 16 + 1];
#pragma unroll
  for (int r = 0; r < WR; ++r)
#pragma unroll
    for (int t = 0; t < MB; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][16 * r + 4 * j + i][16 * t + n] = acc[r][t][i];
  __syncthreads();
  for (int e = threadIdx.x; e < WR * 16 * MB * 16; e += KW * 64) {
    const int tok = e / (WR * 16);
    const int cr = e - tok * (WR * 16);
    const int ch = row0 + cr;
    if (tok >= M || ch >= N) continue;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < KW; ++w) s += red[w][cr][tok];
    if (part != nullptr) {
      part[((int64_t)split * M + tok) * N + ch] = s;
    } else {
      if (bias != nullptr) s += ll_to_f32(bias[ch]);
      Y[(int64_t)tok * ldy + ch] = ll_from_f32<T>(s);
    }
  }
}

template <typename T, typename TO = T>
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                     const T* __restrict__ bias, TO* __restrict__ Y, int64_t ldy,
                                     int M, int N) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)M * N) return;
  const int tok = (int)(e / N), ch = (int)(e - (int64_t)tok * N);
  float s = 0.f;
  for (int sp = 0; sp < splits; ++sp) s += part[((int64_t)sp * M + tok) * N + ch];
  if (bias != nullptr) s += ll_to_f32(bias[ch]);
  Y[(int64_t)tok * ldy + ch] = ll_from_f32<TO>(s);
}

// ---------------------------------------------------------------- tiled
constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLdsStride = kBK + 8;  // elements; 144 B rows

template <typename T>
__global__ __launch_bounds__(256) void gemm_tiled_kernel(const T* __restrict__ X, int64_t ldx,
                                                         const T* __restrict__ W, int64_t ldw,
                                                         const T* __restrict__ bias,
                                                         T* __restrict__ Y, int64_t ldy, int M,
                                                         int N, int K) {
  typedef typename Vec8<T>::type V8;
  __shared__ __attribute__((aligned(16))) T As[kBM * kLdsStride];
  __shared__ __attribute__((aligned(16))) T Bs[kBN * kLdsStride];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, j = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;

  // global -> register staging: 128 rows x 8 chunks of 16 B per operand,
  // 4 chunks per thread per operand
  V8 ra[4], rb[4];
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 3, ch = c & 7;
      const int k = k0 + ch * 8;
      const int gm = m0 + row, gn = n0 + row;
      ra[u] = (gm < M && k < K) ? *(const V8*)(X + (int64_t)gm * ldx + k) : zero8<V8>();
      rb[u] = (gn < N && k < K) ? *(const V8*)(W + (int64_t)gn * ldw + k) : zero8<V8>();
    }
  };
  auto store_stage = [&]() {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 3, ch = c & 7;
      *(V8*)(As + row * kLdsStride + ch * 8) = ra[u];
      *(V8*)(Bs + row * kLdsStride + ch * 8) = rb[u];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int nk = (K + kBK - 1) / kBK;
  load_stage(0);
  store_stage();
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) load_stage((kt + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      V8 av[4], bv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a)
        av[a] = *(const V8*)(As + (wm * 64 + 16 * a + n) * kLdsStride + kk + 8 * j);
#pragma unroll
      for (int b = 0; b < 4; ++b)
        bv[b] = *(const V8*)(Bs + (wn * 64 + 16 * b + n) * kLdsStride + kk + 8 * j);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma16x16x32(av[a], bv[b], acc[a][b]);
    }
    __syncthreads();
    if (kt + 1 < nk) {
      store_stage();
      __syncthreads();
    }
  }
  // acc[a][b][i] = Y[m0 + wm*64 + 16a + 4j + i][n0 + wn*64 + 16b + n]
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int col = n0 + wn * 64 + 16 * b + n;
    if (col >= N) continue;
    const float bb = bias != nullptr ? ll_to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + wm * 64 + 16 * a + 4 * j + i;
        if (row < M) Y[(int64_t)row * ldy + col] = ll_from_f32<T>(acc[a][b][i] + bb);
      }
  }
}

// ---------------------------------------------------------------- fp32
template <typename T>
__global__ __launch_bounds__(256) void gemm_fp32_kernel(const T* __restrict__ X, int64_t ldx,
                                                        const T* __restrict__ W, int64_t ldw,
                                                        const T* __restrict__ bias,
                                                        T* __restrict__ Y, int64_t ldy, int M,
                                                        int N, int K) {
  __shared__ float xs[16][65];
  __shared__ float ws[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int e = threadIdx.x; e < 16 * 64; e += 256) {
      const int r = e >> 4, kk = e & 15;
      const int gm = m0 + r, gn = n0 + r, k = k0 + kk;
      xs[kk][r] = (gm < M && k < K) ? ll_to_f32(X[(int64_t)gm * ldx + k]) : 0.f;
      ws[kk][r] = (gn < N && k < K) ? ll_to_f32(W[(int64_t)gn * ldw + k]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float xr[4], wr[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) xr[a] = xs[kk][ty + 16 * a];
#pragma unroll
      for (int b = 0; b < 4; ++b) wr[b] = ws[kk][tx + 16 * b];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = fmaf(xr[a], wr[b], acc[a][b]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int row = m0 + ty + 16 * a, col = n0 + tx + 16 * b;
      if (row < M && col < N) {
        float v = acc[a][b];
        if (bias != nullptr) v += ll_to_f32(bias[col]);
        Y[(int64_t)row * ldy + col] = ll_from_f32<T>(v);
      }
    }
}

// Kernel choice and split count for M <= 64, from sweeps on MI355X at the
// Qwen2 decode shapes (M = 40): the LDS kernel wins when the weight matrix is
// wide or deep, the direct kernel on the small 2k x 2k projections.
struct SkinnyPlan {
  bool dma;
  int splits;  // K splits across workgroups (all non-empty)
  int ksps;    // 32-wide k-steps per split
  int tr;      // DMA kernel: rows per tile (64, or 128 for wide one-split 16-bit weights)
  int tiles;   // row tiles
  int nst;     // LDS stage buffers of the DMA kernel
  int rotate;  // DMA kernel: rotate the k-chunk order per workgroup
  bool packed; // DMA kernel: W in the ll_gemm_pack layout
};

constexpr int kDirWR = 2, kDirKW = 4, kDirU = 2;

// es: element size in bytes (2 for bf16/fp16, 1 for int8). A stage is a
// 256-byte row chunk: K * es / 256 chunks, four MFMA k-steps each.
SkinnyPlan plan_skinny(int64_t N, int64_t K, int es = 2) {
  SkinnyPlan p;
  p.nst = 2;
  p.rotate = 0;
  p.packed = false;
  p.tr = kDmaTR;
  const int ksteps = (int)((K + 31) / 32);
  p.dma = ((K * es) % 256 == 0);
  if (p.dma) {
    // Measured at the Qwen2.5 decode shapes (M = 40): the weight stream is
    // fastest with about one workgroup per CU when the row tiles are few
    // (split K until tiles * splits reaches 256, three stage buffers) and with
    // one split and two stage buffers (two workgroups per CU) when they are
    // many; rotating each workgroup's k-chunk order spreads the concurrent
    // reads over more HBM channels.
    // With one split and more 64-row tiles than CUs (lm_head), 128-row tiles
    // with three stage buffers (one workgroup per CU) are faster: each
    // activation stage then serves twice the weight rows.
    const int chunks = (int)(K * es / 256);
    p.tiles = (int)((N + kDmaTR - 1) / kDmaTR);
    int sp = 256 / p.tiles;
    if (sp > chunks / 2) sp = chunks / 2;
    if (sp < 1) sp = 1;
    const int per = (chunks + sp - 1) / sp;
    p.splits = (chunks + per - 1) / per;
    p.ksps = per * 4;
    p.nst = (p.tiles * p.splits <= 256) ? 3 : 2;
    p.rotate = 1;
    if (p.splits == 1 && p.tiles > 256) {
      p.tr = 128;
      p.tiles = (int)((N + 127) / 128);
      p.nst = 3;
    }
  } else {
    p.tiles = (int)((N + 16 * kDirWR - 1) / (16 * kDirWR));
    int sp = 1;
    while ((int64_t)p.tiles * sp < 512 && ksteps / (sp * 2) >= kDirKW * 2) sp *= 2;
    const int per = (ksteps + sp - 1) / sp;
    p.splits = (ksteps + per - 1) / per;
    p.ksps = per;
  }
  return p;
}

// Tile height of the fused gate/up kernel (one split): the lowest of 64, 96
// and 128 rows (half gate, half up channels) whose tiles fit in one dispatch
// round of the 256 CUs. At the Qwen2.5-3B shape (I = 11008) 96-row tiles give
// 230 workgroups (128-row tiles: 172, leaving a third of the CUs idle): 17.45
// against 18.2 us per bf16 launch with cold weights, three stage buffers (four
// measured 17.8).
int gate_up_tr(int64_t I) {
  if (ll_cdiv(I, 32) <= 256) return 64;
  return ll_cdiv(I, 48) <= 256 ? 96 : 128;
}

template <typename T, int MB, typename TO = T>
void launch_skinny_mb(const SkinnyPlan& p, const T* X, int64_t ldx, const T* W, int64_t ldw,
                      const T* bias, T* Y, int64_t ldy, float* part, int M, int N, int K,
                      hipStream_t stream) {
  const dim3 grid((unsigned)p.tiles, (unsigned)p.splits);
  if (p.dma) {
    const size_t lds = (size_t)p.nst * (p.tr + 16 * MB) * 256;
#define LL_DMA_LAUNCH(S, PKD, TR_)                                                              \
  hipLaunchKernelGGL((gemm_dma_kernel<T, MB, S, PKD, 0, TR_, TO>), grid, dim3(256), lds, stream, X, \
                     ldx, W, ldw, M, N, K, p.ksps, p.rotate, bias, Y, ldy, part, I8Epi{})
    if (p.tr == 128) {
      if (p.packed) LL_DMA_LAUNCH(3, true, 128); else LL_DMA_LAUNCH(3, false, 128);
      return;
    }
    if (p.packed) {
      if (p.nst == 3) LL_DMA_LAUNCH(3, true, 64); else LL_DMA_LAUNCH(2, true, 64);
    } else {
      if (p.nst == 3) LL_DMA_LAUNCH(3, false, 64); else LL_DMA_LAUNCH(2, false, 64);
    }
#undef LL_DMA_LAUNCH
  } else if constexpr (sizeof(T) == 2 && std::is_same<T, TO>::value) {
    hipLaunchKernelGGL((gemm_direct_kernel<T, MB, kDirWR, kDirKW, kDirU>), grid,
                       dim3(64 * kDirKW), 0, stream, X, ldx, W, ldw, bias, Y, ldy, part, M, N, K,
                       p.ksps);
  }
}

template <typename T, typename TO = T>
void launch_skinny(const SkinnyPlan& p, const T* X, int64_t ldx, const T* W, int64_t ldw,
                   const T* bias, T* Y, int64_t ldy, float* part, int M, int N, int K,
                   hipStream_t stream) {
  switch ((M + 15) / 16) {
    case 1: launch_skinny_mb<T, 1, TO>(p, X, ldx, W, ldw, bias, Y, ldy, part, M, N, K, stream); break;
    case 2: launch_skinny_mb<T, 2, TO>(p, X, ldx, W, ldw, bias, Y, ldy, part, M, N, K, stream); break;
    case 3: launch_skinny_mb<T, 3, TO>(p, X, ldx, W, ldw, bias, Y, ldy, part, M, N, K, stream); break;
    default: launch_skinny_mb<T, 4, TO>(p, X, ldx, W, ldw, bias, Y, ldy, part, M, N, K, stream); break;
  }
}

template <typename T>
int launch_gemm(const T* X, int64_t ldx, const T* W, int64_t ldw, const T* bias, T* Y, int64_t ldy,
                int64_t M, int64_t N, int64_t K, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (M <= 64) {
    const SkinnyPlan p = plan_skinny(N, K);
    float* part = nullptr;
    if (p.splits > 1) {
      const int64_t need = (int64_t)p.splits * M * N * 4;
      LL_CHECK_ARG(ws != nullptr && ws_bytes >= need,
                   "ll_gemm: workspace too small (need %lld bytes)", (long long)need);
      part = (float*)ws;
    }
    launch_skinny<T>(p, X, ldx, W, ldw, bias, Y, ldy, part, (int)M, (int)N, (int)K, stream);
    if (p.splits > 1) {
      const int64_t total = M * N;
      hipLaunchKernelGGL((splitk_reduce_kernel<T>), dim3((unsigned)((total + 255) / 256)), dim3(256),
                         0, stream, part, p.splits, bias, Y, ldy, (int)M, (int)N);
    }
    LL_RETURN_LAUNCH();
  }
  // above 64 rows: the 256 x 256 MFMA tile kernel (gemm_tiles.hip) wherever
  // its layout constraints hold, else the 128 x 128 kernel below
  constexpr int dt = sizeof(T) == 2 && !__is_same(T, __bf16) ? LL_F16 : LL_BF16;
  if (ll_gemm_tiled_supported(M, N, K, dt) && ldy % 4 == 0 && ((uintptr_t)Y) % 8 == 0 &&
      (ldx * 2) % 16 == 0 && (ldw * 2) % 16 == 0 && (((uintptr_t)X | (uintptr_t)W) % 16) == 0)
    return ll_gemm_tiled(X, ldx, W, ldw, bias, Y, ldy, M, N, K, dt, stream);
  const dim3 grid((unsigned)ll_cdiv(N, kBN), (unsigned)ll_cdiv(M, kBM));
  hipLaunchKernelGGL((gemm_tiled_kernel<T>), grid, dim3(256), 0, stream, X, ldx, W, ldw, bias, Y,
                     ldy, (int)M, (int)N, (int)K);
  LL_RETURN_LAUNCH();
}

}  // namespace

extern "C" int64_t ll_gemm_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M > 64) return 0;
  const SkinnyPlan p = plan_skinny(N, K);
  return p.splits > 1 ? (int64_t)p.splits * M * N * 4 : 0;
}

extern "C" int ll_gemm_splitk_count(int64_t M, int64_t N, int64_t K) {
  if (M > 64 || M <= 0) return 0;
  return plan_skinny(N, K).splits;
}

namespace {

int gemm_splitk_impl(const char* name, const void* X, int64_t ldx, const void* W, int64_t ldw,
                     int64_t M, int64_t N, int64_t K, int dtype, float* part, int64_t part_bytes,
                     bool packed, hipStream_t stream) {
  LL_CHECK_ARG(X && W && part, "%s: null pointer", name);
  LL_CHECK_ARG(M > 0 && M <= 64 && N > 0 && K > 0, "%s: needs 0 < M <= 64 (M=%lld)", name,
               (long long)M);
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "%s: bf16/fp16 only", name);
  LL_CHECK_ARG(K % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0,
               "%s: K and leading dims must be multiples of 8", name);
  LL_CHECK_ARG((((uintptr_t)X | (uintptr_t)W) % 16) == 0, "%s: X and W must be 16 B aligned", name);
  SkinnyPlan p = plan_skinny(N, K);
  if (packed) {
    LL_CHECK_ARG(p.dma, "%s: packed weights need K %% %d == 0", name, kDmaKC);
    p.packed = true;
    p.rotate = 0;  // neighbouring workgroups stream neighbouring blocks
  }
  LL_CHECK_ARG(part_bytes >= (int64_t)p.splits * M * N * 4,
               "%s: partial buffer too small (need %lld bytes)", name,
               (long long)((int64_t)p.splits * M * N * 4));
  if (dtype == LL_BF16)
    launch_skinny<__bf16>(p, (const __bf16*)X, ldx, (const __bf16*)W, ldw, nullptr, nullptr, 0,
                          part, (int)M, (int)N, (int)K, stream);
  else
    launch_skinny<_Float16>(p, (const _Float16*)X, ldx, (const _Float16*)W, ldw, nullptr, nullptr,
                            0, part, (int)M, (int)N, (int)K, stream);
  LL_RETURN_LAUNCH();
}

}  // namespace

extern "C" int ll_gemm_splitk(const void* X, int64_t ldx, const void* W, int64_t ldw, int64_t M,
                              int64_t N, int64_t K, int dtype, float* part, int64_t part_bytes,
                              hipStream_t stream) {
  return gemm_splitk_impl("ll_gemm_splitk", X, ldx, W, ldw, M, N, K, dtype, part, part_bytes,
                          false, stream);
}

extern "C" int ll_gemm_packed_tile_rows(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % kDmaKC != 0) return 0;
  return plan_skinny(N, K).tr;
}

extern "C" int ll_gemm_packed_gate_up_tile_rows(int64_t I) {
  return I > 0 ? gate_up_tr(I) : 0;
}

extern "C" int64_t ll_gemm_packed_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % kDmaKC != 0) return 0;
  const int tr = plan_skinny(N, K).tr;
  return ll_cdiv(N, tr) * tr * K * 2;
}

extern "C" int ll_gemm_pack(const void* W, int64_t ldw, int64_t N, int64_t K, int dtype, void* Wp,
                            int64_t wp_bytes, hipStream_t stream) {
  LL_CHECK_ARG(W && Wp, "ll_gemm_pack: null pointer");
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "ll_gemm_pack: bf16/fp16 only");
  LL_CHECK_ARG(N > 0 && K > 0 && K % kDmaKC == 0, "ll_gemm_pack: needs K %% %d == 0 (K=%lld)",
               kDmaKC, (long long)K);
  LL_CHECK_ARG(ldw >= K && ldw % 8 == 0 && ((uintptr_t)W | (uintptr_t)Wp) % 16 == 0,
               "ll_gemm_pack: W rows must be 16 B aligned");
  const int64_t bytes = ll_gemm_packed_bytes(N, K);
  LL_CHECK_ARG(wp_bytes >= bytes, "ll_gemm_pack: output too small (need %lld bytes)",
               (long long)bytes);
  const int64_t units = bytes / 16;
  const int tr = plan_skinny(N, K).tr;
  const int tiles = (int)ll_cdiv(N, tr);
  hipLaunchKernelGGL(gemm_pack_kernel, dim3((unsigned)ll_cdiv(units, 256)), dim3(256), 0, stream,
                     (const u32x4*)W, ldw / 8, (u32x4*)Wp, (int)N, tiles, units, 0, tr);
  LL_RETURN_LAUNCH();
}

extern "C" int64_t ll_gemm_packed_gate_up_bytes(int64_t I, int64_t K) {
  if (I <= 0 || K <= 0 || K % kDmaKC != 0) return 0;
  const int tr = gate_up_tr(I);
  return ll_cdiv(I, tr / 2) * tr * K * 2;
}

extern "C" int ll_gemm_pack_gate_up(const void* W, int64_t ldw, int64_t I, int64_t K, int dtype,
                                    void* Wp, int64_t wp_bytes, hipStream_t stream) {
  LL_CHECK_ARG(W && Wp, "ll_gemm_pack_gate_up: null pointer");
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "ll_gemm_pack_gate_up: bf16/fp16 only");
  LL_CHECK_ARG(I > 0 && K > 0 && K % kDmaKC == 0,
               "ll_gemm_pack_gate_up: needs K %% %d == 0 (K=%lld)", kDmaKC, (long long)K);
  LL_CHECK_ARG(ldw >= K && ldw % 8 == 0 && ((uintptr_t)W | (uintptr_t)Wp) % 16 == 0,
               "ll_gemm_pack_gate_up: W rows must be 16 B aligned");
  const int64_t bytes = ll_gemm_packed_gate_up_bytes(I, K);
  LL_CHECK_ARG(wp_bytes >= bytes, "ll_gemm_pack_gate_up: output too small (need %lld bytes)",
               (long long)bytes);
  const int64_t units = bytes / 16;
  const int tr = gate_up_tr(I);
  const int tiles = (int)ll_cdiv(I, tr / 2);
  hipLaunchKernelGGL(gemm_pack_kernel, dim3((unsigned)ll_cdiv(units, 256)), dim3(256), 0, stream,
                     (const u32x4*)W, ldw / 8, (u32x4*)Wp, (int)(2 * I), tiles, units, (int)I, tr);
  LL_RETURN_LAUNCH();
}

extern "C" int ll_gemm_gate_up_silu_packed(const void* X, int64_t ldx, const void* Wp, int64_t M,
                                           int64_t I, int64_t K, int dtype, void* act,
                                           int64_t ld_act, hipStream_t stream) {
  LL_CHECK_ARG(X && Wp && act, "ll_gemm_gate_up_silu_packed: null pointer");
  LL_CHECK_ARG(M > 0 && M <= 64 && I > 0 && K > 0 && K % kDmaKC == 0,
               "ll_gemm_gate_up_silu_packed: needs 0 < M <= 64 and K %% %d == 0", kDmaKC);
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "ll_gemm_gate_up_silu_packed: bf16/fp16 only");
  LL_CHECK_ARG(ldx % 8 == 0 && (((uintptr_t)X | (uintptr_t)Wp) % 16) == 0,
               "ll_gemm_gate_up_silu_packed: X rows must be 16 B aligned");
  const int tr = gate_up_tr(I);
  const int tiles = (int)ll_cdiv(I, tr / 2);
  const int nst = (tr != 64 || tiles <= 256) ? 3 : 2;
  const int ksps = (int)(K / 32);
  auto run = [&](auto tag) {
    typedef decltype(tag) T;
    const T* x = (const T*)X;
    const T* w = (const T*)Wp;
    T* y = (T*)act;
    const dim3 grid((unsigned)tiles, 1);
#define LL_GU(MB_)                                                                              \
  do {                                                                                          \
    const size_t lds = (size_t)nst * (tr + 16 * MB_) * kDmaKC * 2;                              \
    if (tr == 96)                                                                               \
      hipLaunchKernelGGL((gemm_dma_kernel<T, MB_, 3, true, 1, 96>), grid, dim3(256), lds,        \
                         stream, x, ldx, w, K, (int)M, (int)(2 * I), (int)K, ksps, 0, nullptr, y, \
                         ld_act, nullptr, I8Epi{});                                             \
    else if (tr == 128)                                                                         \
      hipLaunchKernelGGL((gemm_dma_kernel<T, MB_, 3, true, 1, 128>), grid, dim3(256), lds,       \
                         stream, x, ldx, w, K, (int)M, (int)(2 * I), (int)K, ksps, 0, nullptr, y, \
                         ld_act, nullptr, I8Epi{});                                             \
    else if (nst == 3)                                                                          \
      hipLaunchKernelGGL((gemm_dma_kernel<T, MB_, 3, true, 1>), grid, dim3(256), lds, stream, x, \
                         ldx, w, K, (int)M, (int)(2 * I), (int)K, ksps, 0, nullptr, y, ld_act,  \
                         nullptr, I8Epi{});                                                     \
    else                                                                                        \
      hipLaunchKernelGGL((gemm_dma_kernel<T, MB_, 2, true, 1>), grid, dim3(256), lds, stream, x, \
                         ldx, w, K, (int)M, (int)(2 * I), (int)K, ksps, 0, nullptr, y, ld_act,  \
                         nullptr, I8Epi{});                                                     \
  } while (0)
    switch ((M + 15) / 16) {
      case 1: LL_GU(1); break;
      case 2: LL_GU(2); break;
      case 3: LL_GU(3); break;
      default: LL_GU(4); break;
    }
#undef LL_GU
  };
  if (dtype == LL_BF16) run(__bf16{}); else run(_Float16{});
  LL_RETURN_LAUNCH();
}

extern "C" int ll_gemm_splitk_packed(const void* X, int64_t ldx, const void* Wp, int64_t M,
                                     int64_t N, int64_t K, int dtype, float* part,
                                     int64_t part_bytes, hipStream_t stream) {
  return gemm_splitk_impl("ll_gemm_splitk_packed", X, ldx, Wp, K, M, N, K, dtype, part,
                          part_bytes, true, stream);
}

namespace {
// The packed-weight GEMM for M <= 64 with output type TO (the model dtype,
// or fp32 for logits that are argmaxed unrounded).
int gemm_packed_impl(const char* name, const void* X, int64_t ldx, const void* Wp,
                     const void* bias, void* Y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                     int dtype, bool out_f32, void* workspace, int64_t workspace_bytes,
                     hipStream_t stream) {
  LL_CHECK_ARG(X && Wp && Y, "%s: null pointer", name);
  LL_CHECK_ARG(M > 0 && M <= 64 && N > 0 && K > 0 && K % kDmaKC == 0,
               "%s: needs 0 < M <= 64 and K %% %d == 0", name, kDmaKC);
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "%s: bf16/fp16 only", name);
  LL_CHECK_ARG(ldx % 8 == 0 && (((uintptr_t)X | (uintptr_t)Wp) % 16) == 0,
               "%s: X rows must be 16 B aligned", name);
  LL_CHECK_ARG(ldx >= K && ldy >= N, "%s: row strides shorter than the rows", name);
  SkinnyPlan p = plan_skinny(N, K);
  p.packed = true;
  p.rotate = 0;
  float* part = nullptr;
  if (p.splits > 1) {
    const int64_t need = (int64_t)p.splits * M * N * 4;
    LL_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                 "%s: workspace too small (need %lld bytes)", name, (long long)need);
    part = (float*)workspace;
  }
  auto run = [&](auto tag, auto otag) {
    typedef decltype(tag) T;
    typedef decltype(otag) TO;
    launch_skinny<T, TO>(p, (const T*)X, ldx, (const T*)Wp, K, (const T*)bias, (T*)Y, ldy, part,
                         (int)M, (int)N, (int)K, stream);
    if (p.splits > 1) {
      const int64_t total = M * N;
      hipLaunchKernelGGL((splitk_reduce_kernel<T, TO>), dim3((unsigned)((total + 255) / 256)),
                         dim3(256), 0, stream, part, p.splits, (const T*)bias, (TO*)Y, ldy, (int)M,
                         (int)N);
    }
  };
  if (dtype == LL_BF16) {
    if (out_f32) run(__bf16{}, float{}); else run(__bf16{}, __bf16{});
  } else {
    if (out_f32) run(_Float16{}, float{}); else run(_Float16{}, _Float16{});
  }
  LL_RETURN_LAUNCH();
}
}  // namespace

extern "C" int ll_gemm_packed(const void* X, int64_t ldx, const void* Wp, const void* bias, void* Y,
                              int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype,
                              void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  return gemm_packed_impl("ll_gemm_packed", X, ldx, Wp, bias, Y, ldy, M, N, K, dtype, false,
                          workspace, workspace_bytes, stream);
}

extern "C" int ll_gemm_packed_f32(const void* X, int64_t ldx, const void* Wp, const void* bias,
                                  float* Y, int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype,
                                  void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  return gemm_packed_impl("ll_gemm_packed_f32", X, ldx, Wp, bias, Y, ldy, M, N, K, dtype, true,
                          workspace, workspace_bytes, stream);
}

namespace {
// Persistent form of the packed GEMM with the argmax epilogue, for the plans
// with 128-row tiles and one split (the lm_head): at most one workgroup per
// CU (kLmCUs), each taking tiles blockIdx.x, blockIdx.x + gridDim.x, ...; its
// LDS copy ring runs on from one tile into the next, so the next tile's first
// stages are in flight while a tile is finished and stored, where a workgroup
// per tile pays the first copies' round trip and its ramp once per tile. The
// epilogue is EPI 2's (the tile's logits and per-token (value, first index))
// with buffer stores: every wave issues the same number of them for every
// tile (a masked lane's offset lies past the buffer), so the ring's vmcnt
// waits count them: for two iterations after an epilogue its stores sit
// among the copies in flight. No bias (the lm_head has none).
constexpr int kLmCUs = 256;
constexpr int kLmStages = 3;
constexpr uint32_t kLmNoStore = 0x80000000u;

template <typename T, int MB>
__global__ __launch_bounds__(256) void lm_head_argmax_kernel(const T* __restrict__ X, int64_t ldx,
                                                             const T* __restrict__ Wp,
                                                             float* __restrict__ Y, int64_t ldy,
                                                             int M, int N, int K, int tiles,
                                                             float* __restrict__ am_val,
                                                             int* __restrict__ am_idx) {
  typedef typename Vec8<T>::type V8;
  constexpr int TR = 128, NST = kLmStages, RB = 2, XR = 16 * MB;
  constexpr int KC = 128, CE = 8, KSTEP = 32;
  constexpr int ROWB = 256, CH = 16, RPI = 4;
  constexpr int W_PER_WAVE = (TR / RPI) / 4;
  constexpr int X_PER_WAVE = (XR / RPI) / 4;
  constexpr int C = W_PER_WAVE + X_PER_WAVE;  // copies per wave per stage
  constexpr int SY = RB * MB;                 // logit stores per wave per tile
  constexpr int STAGE_B = (TR + XR) * ROWB;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  float* sval = (float*)(smem + NST * STAGE_B);  // the epilogue's rows, outside the ring
  int* sidx = (int*)(sval + 4 * XR);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, j = lane >> 4;
  const int lr_in = lane / CH, p = lane % CH;
  const int nst = K / KC;
  const int my_tiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int total = my_tiles * nst;  // stages of this workgroup, tile after tile
  const __amdgpu_buffer_rsrc_t yres =
      __builtin_amdgcn_make_buffer_rsrc(Y, (short)0, (int)((int64_t)M * ldy * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t vres =
      __builtin_amdgcn_make_buffer_rsrc(am_val, (short)0, M * tiles * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t ires =
      __builtin_amdgcn_make_buffer_rsrc(am_idx, (short)0, M * tiles * 4, 0x00020000);
  auto issue = [&](int g) {  // stage g: k chunk g % nst of this workgroup's tile g / nst
    const int jt = g / nst, kc = g - jt * nst;
    const int tile = (int)blockIdx.x + jt * (int)gridDim.x;
    char* base = smem + (g % NST) * STAGE_B;
#pragma unroll
    for (int q = 0; q < W_PER_WAVE; ++q) {
      const int ii = wave * W_PER_WAVE + q;
      const char* gp = (const char*)Wp + ((int64_t)kc * tiles + tile) * (TR * ROWB) + ii * 1024 +
                       lane * 16;
      dma16_stream(gp, base + ii * 1024);
    }
#pragma unroll
    for (int q = 0; q < X_PER_WAVE; ++q) {
      const int ii = wave + q * 4;
      const int r = ii * RPI + lr_in;
      const T* gp = X + (int64_t)min(r, M - 1) * ldx + kc * KC + (p ^ (r & 15)) * CE;
      dma16(gp, base + TR * ROWB + ii * 1024);
    }
  };
  f32x4 acc[RB][MB];
#pragma unroll
  for (int b = 0; b < RB; ++b)
#pragma unroll
    for (int t = 0; t < MB; ++t) acc[b][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // acc[b][t][i] = Y[token 16t + n][channel 128 tile + 32 wave + 16 b + 4 j + i]
  auto epilogue = [&](int tile) {
    float bv[MB];
    int bi[MB];
#pragma unroll
    for (int t = 0; t < MB; ++t) { bv[t] = -INFINITY; bi[t] = 0x7fffffff; }
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const int ch = tile * TR + wave * 16 * RB + 16 * b + 4 * j;
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        const int tok = 16 * t + n;
        const f32x4 v = acc[b][t];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // channel indices rise with (b, i), so a tie keeps the earlier pick
          const bool take = (ch + i < N) & ((v[i] > bv[t]) | ((v[i] == bv[t]) & (bi[t] == 0x7fffffff)));
          bv[t] = take ? v[i] : bv[t];
          bi[t] = take ? ch + i : bi[t];
        }
        const uint32_t off = (tok < M && ch < N) ? (uint32_t)(((int64_t)tok * ldy + ch) * 4) : kLmNoStore;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), yres, off, 0, 0);
        asm volatile("" ::: "memory");
      }
    }
#pragma unroll
    for (int t = 0; t < MB; ++t) {
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        const float ov = __shfl_xor(bv[t], o, 64);
        const int oi = __shfl_xor(bi[t], o, 64);
        const bool take = (ov > bv[t]) | ((ov == bv[t]) & (oi < bi[t]));
        bv[t] = take ? ov : bv[t];
        bi[t] = take ? oi : bi[t];
      }
    }
    if (j == 0) {
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        sval[wave * XR + 16 * t + n] = bv[t];
        sidx[wave * XR + 16 * t + n] = bi[t];
      }
    }
    lds_barrier();
    if (wave == 0) {  // lane = token: its value and index over the four waves
      const int tok = min(lane, XR - 1);
      float v = sval[tok];
      int i = sidx[tok];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const float ov = sval[w * XR + tok];
        const int oi = sidx[w * XR + tok];
        const bool take = (ov > v) | ((ov == v) & (oi < i));
        v = take ? ov : v;
        i = take ? oi : i;
      }
      const uint32_t off = lane < M ? (uint32_t)((lane * tiles + tile) * 4) : kLmNoStore;
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), vres, off, 0, 0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_raw_buffer_store_b32((uint32_t)i, ires, off, 0, 0);
      asm volatile("" ::: "memory");
    }
  };
#pragma unroll
  for (int g = 0; g < NST - 1; ++g)
    if (g < total) issue(g);
  int last_ep = -NST;  // the iteration of the last epilogue
  for (int g = 0; g < total; ++g) {
    // stage g's copies are done; stage g + 1's may stay in flight, and so may
    // the last epilogue's stores while they are younger than stage g's copies
    const bool later = g + 1 < total;
    if (g - last_ep <= 2) {
      if (wave == 0) {
        if (later) vm_wait<C + SY + 2>(); else vm_wait<SY + 2>();
      } else {
        if (later) vm_wait<C + SY>(); else vm_wait<SY>();
      }
    } else {
      if (later) vm_wait<C>(); else vm_wait<0>();
    }
    lds_barrier();  // and every wave is done with stage g - 1, refilled here
    if (g + NST - 1 < total) issue(g + NST - 1);
    const char* wb = smem + (g % NST) * STAGE_B;
    const char* xb = wb + TR * ROWB;
#pragma unroll
    for (int s = 0; s < KC / KSTEP; ++s) {
      V8 a[RB];
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int lr = wave * 16 * RB + 16 * b + n;
        a[b] = *(const V8*)(wb + lr * ROWB + (((4 * s + j) ^ (lr & 15)) * 16));
      }
#pragma unroll
      for (int t = 0; t < MB; ++t) {
        const int xr = 16 * t + n;
        const V8 xv = *(const V8*)(xb + xr * ROWB + (((4 * s + j) ^ (xr & 15)) * 16));
#pragma unroll
        for (int b = 0; b < RB; ++b) acc[b][t] = mfma16x16x32(a[b], xv, acc[b][t]);
      }
    }
    if (g % nst == nst - 1) {
      epilogue((int)blockIdx.x + (g / nst) * (int)gridDim.x);
#pragma unroll
      for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int t = 0; t < MB; ++t) acc[b][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
      last_ep = g;
    }
  }
}

// The packed GEMM with the EPI 2 epilogue (fp32 output + the argmax's first
// pass); one-split plans only. 128-row plans without bias run persistent.
template <typename T, int MB>
void launch_argmax_mb(const SkinnyPlan& p, const T* X, int64_t ldx, const T* Wp, const T* bias,
                      float* Y, int64_t ldy, int M, int N, int K, float* am_val, int* am_idx,
                      hipStream_t stream) {
  if (p.tr == 128 && bias == nullptr && N % 4 == 0 && ldy % 4 == 0 &&
      ((uintptr_t)Y % 16) == 0 && (int64_t)M * ldy * 4 < ((int64_t)1 << 31)) {
    const int grid = p.tiles < kLmCUs ? p.tiles : kLmCUs;
    const size_t lds = (size_t)kLmStages * (128 + 16 * MB) * 256 + 4 * 16 * MB * 8;
    hipLaunchKernelGGL((lm_head_argmax_kernel<T, MB>), dim3((unsigned)grid), dim3(256), lds,
                       stream, X, ldx, Wp, Y, ldy, M, N, K, p.tiles, am_val, am_idx);
    return;
  }
  const dim3 grid((unsigned)p.tiles, 1u);
  const size_t lds = (size_t)p.nst * (p.tr + 16 * MB) * 256;
  I8Epi e{};
  e.am_val = am_val;
  e.am_idx = am_idx;
#define LL_AM_LAUNCH(S, TR_)                                                                      \
  hipLaunchKernelGGL((gemm_dma_kernel<T, MB, S, true, 2, TR_, float>), grid, dim3(256), lds,       \
                     stream, X, ldx, Wp, (int64_t)K, M, N, K, p.ksps, 0, bias, (T*)(void*)Y, ldy,  \
                     nullptr, e)
  if (p.tr == 128) LL_AM_LAUNCH(3, 128);
  else if (p.nst == 3) LL_AM_LAUNCH(3, 64);
  else LL_AM_LAUNCH(2, 64);
#undef LL_AM_LAUNCH
}
}  // namespace

extern "C" int64_t ll_gemm_packed_f32_argmax_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || M > 64 || N <= 0 || K <= 0 || K % kDmaKC != 0) return 0;
  const SkinnyPlan p = plan_skinny(N, K);
  if (p.splits == 1) return M * p.tiles * 8;
  return (int64_t)p.splits * M * N * 4 + ll_argmax_workspace_size(M, N);
}

extern "C" int ll_gemm_packed_f32_argmax(const void* X, int64_t ldx, const void* Wp,
                                         const void* bias, float* Y, int64_t ldy, int64_t M,
                                         int64_t N, int64_t K, int dtype, int64_t* tokens,
                                         const uint32_t* status, void* workspace,
                                         int64_t workspace_bytes, hipStream_t stream) {
  const char* name = "ll_gemm_packed_f32_argmax";
  LL_CHECK_ARG(X && Wp && Y && tokens, "%s: null pointer", name);
  LL_CHECK_ARG(M > 0 && M <= 64 && N > 0 && K > 0 && K % kDmaKC == 0,
               "%s: needs 0 < M <= 64 and K %% %d == 0", name, kDmaKC);
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "%s: bf16/fp16 only", name);
  LL_CHECK_ARG(ldx % 8 == 0 && (((uintptr_t)X | (uintptr_t)Wp) % 16) == 0,
               "%s: X rows must be 16 B aligned", name);
  LL_CHECK_ARG(ldx >= K && ldy >= N, "%s: row strides shorter than the rows", name);
  const int64_t need = ll_gemm_packed_f32_argmax_workspace_size(M, N, K);
  LL_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
               "%s: workspace too small (need %lld bytes)", name, (long long)need);
  SkinnyPlan p = plan_skinny(N, K);
  p.packed = true;
  p.rotate = 0;
  if (p.splits > 1) {
    // a plan with k splits: the GEMM and a separate argmax
    const int64_t part_bytes = (int64_t)p.splits * M * N * 4;
    const int rc = gemm_packed_impl(name, X, ldx, Wp, bias, Y, ldy, M, N, K, dtype, true,
                                    workspace, part_bytes, stream);
    if (rc != LL_OK) return rc;
    void* aws = (char*)workspace + part_bytes;
    const int64_t awsb = workspace_bytes - part_bytes;
    return status != nullptr
               ? ll_argmax_status(Y, ldy, M, N, tokens, aws, awsb, LL_F32, status, stream)
               : ll_argmax(Y, ldy, M, N, tokens, aws, awsb, LL_F32, stream);
  }
  float* am_val = (float*)workspace;
  int* am_idx = (int*)(am_val + M * p.tiles);
  auto run = [&](auto tag) {
    typedef decltype(tag) T;
    switch ((M + 15) / 16) {
      case 1: launch_argmax_mb<T, 1>(p, (const T*)X, ldx, (const T*)Wp, (const T*)bias, Y, ldy, (int)M, (int)N, (int)K, am_val, am_idx, stream); break;
      case 2: launch_argmax_mb<T, 2>(p, (const T*)X, ldx, (const T*)Wp, (const T*)bias, Y, ldy, (int)M, (int)N, (int)K, am_val, am_idx, stream); break;
      case 3: launch_argmax_mb<T, 3>(p, (const T*)X, ldx, (const T*)Wp, (const T*)bias, Y, ldy, (int)M, (int)N, (int)K, am_val, am_idx, stream); break;
      default: launch_argmax_mb<T, 4>(p, (const T*)X, ldx, (const T*)Wp, (const T*)bias, Y, ldy, (int)M, (int)N, (int)K, am_val, am_idx, stream); break;
    }
  };
  if (dtype == LL_BF16) run(__bf16{}); else run(_Float16{});
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    ll_set_error("%s: launch failed: %s", name, hipGetErrorString(e));
    return LL_ERR_HIP;
  }
  return ll_argmax_finish(am_val, am_idx, M, p.tiles, tokens, status, stream);
}

extern "C" int ll_gemm(const void* X, int64_t ldx, const void* W, int64_t ldw, const void* bias,
                       void* Y, int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype,
                       void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  LL_CHECK_ARG(X && W && Y, "ll_gemm: null pointer");
  LL_CHECK_ARG(M >= 0 && N > 0 && K > 0, "ll_gemm: bad shape M=%lld N=%lld K=%lld", (long long)M,
               (long long)N, (long long)K);
  if (M == 0) return LL_OK;
  if (dtype == LL_F32) {
    const dim3 grid((unsigned)ll_cdiv(N, 64), (unsigned)ll_cdiv(M, 64));
    hipLaunchKernelGGL((gemm_fp32_kernel<float>), grid, dim3(256), 0, stream, (const float*)X, ldx,
                       (const float*)W, ldw, (const float*)bias, (float*)Y, ldy, (int)M, (int)N,
                       (int)K);
    LL_RETURN_LAUNCH();
  }
  LL_CHECK_ARG(K % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0,
               "ll_gemm: K and leading dims must be multiples of 8 for %s",
               dtype == LL_BF16 ? "bf16" : "fp16");
  LL_CHECK_ARG((((uintptr_t)X | (uintptr_t)W) % 16) == 0, "ll_gemm: X and W must be 16 B aligned");
  if (dtype == LL_BF16)
    return launch_gemm<__bf16>((const __bf16*)X, ldx, (const __bf16*)W, ldw, (const __bf16*)bias,
                               (__bf16*)Y, ldy, M, N, K, workspace, workspace_bytes, stream);
  if (dtype == LL_F16)
    return launch_gemm<_Float16>((const _Float16*)X, ldx, (const _Float16*)W, ldw,
                                 (const _Float16*)bias, (_Float16*)Y, ldy, M, N, K, workspace,
                                 workspace_bytes, stream);
  ll_set_error("ll_gemm: unsupported dtype %d", dtype);
  return LL_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------- int8 (W8A8)
// Weight streaming with int8 weights and per-token int8 activations, exact
// int32 partial sums (no reference counterpart: the reference's W8A8 module
// quantize/smooth_quant/layer.py:19-59 has no forward; this is its runtime).

extern "C" int64_t ll_gemm_i8_packed_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % 256 != 0) return 0;
  const int tr = plan_skinny(N, K, 1).tr;
  return ll_cdiv(N, tr) * tr * K;
}

extern "C" int ll_gemm_i8_pack(const int8_t* Wq, int64_t ldw, int64_t N, int64_t K, void* Wp,
                               int64_t wp_bytes, hipStream_t stream) {
  LL_CHECK_ARG(Wq && Wp, "ll_gemm_i8_pack: null pointer");
  LL_CHECK_ARG(N > 0 && K > 0 && K % 256 == 0, "ll_gemm_i8_pack: needs K %% 256 == 0 (K=%lld)",
               (long long)K);
  LL_CHECK_ARG(ldw >= K && ldw % 16 == 0 && ((uintptr_t)Wq | (uintptr_t)Wp) % 16 == 0,
               "ll_gemm_i8_pack: W rows must be 16 B aligned");
  const int64_t bytes = ll_gemm_i8_packed_bytes(N, K);
  LL_CHECK_ARG(wp_bytes >= bytes, "ll_gemm_i8_pack: output too small (need %lld bytes)",
               (long long)bytes);
  const int64_t units = bytes / 16;
  hipLaunchKernelGGL(gemm_pack_kernel, dim3((unsigned)ll_cdiv(units, 256)), dim3(256), 0, stream,
                     (const u32x4*)Wq, ldw / 16, (u32x4*)Wp, (int)N,
                     (int)ll_cdiv(N, plan_skinny(N, K, 1).tr), units, 0, plan_skinny(N, K, 1).tr);
  LL_RETURN_LAUNCH();
}

extern "C" int64_t ll_gemm_i8_packed_gate_up_bytes(int64_t I, int64_t K) {
  if (I <= 0 || K <= 0 || K % 256 != 0) return 0;
  const int tr = gate_up_tr(I);
  return ll_cdiv(I, tr / 2) * tr * K;
}

extern "C" int ll_gemm_i8_pack_gate_up(const int8_t* Wq, int64_t ldw, int64_t I, int64_t K,
                                       void* Wp, int64_t wp_bytes, hipStream_t stream) {
  LL_CHECK_ARG(Wq && Wp, "ll_gemm_i8_pack_gate_up: null pointer");
  LL_CHECK_ARG(I > 0 && K > 0 && K % 256 == 0,
               "ll_gemm_i8_pack_gate_up: needs K %% 256 == 0 (K=%lld)", (long long)K);
  LL_CHECK_ARG(ldw >= K && ldw % 16 == 0 && ((uintptr_t)Wq | (uintptr_t)Wp) % 16 == 0,
               "ll_gemm_i8_pack_gate_up: W rows must be 16 B aligned");
  const int64_t bytes = ll_gemm_i8_packed_gate_up_bytes(I, K);
  LL_CHECK_ARG(wp_bytes >= bytes, "ll_gemm_i8_pack_gate_up: output too small (need %lld bytes)",
               (long long)bytes);
  const int64_t units = bytes / 16;
  const int tr = gate_up_tr(I);
  hipLaunchKernelGGL(gemm_pack_kernel, dim3((unsigned)ll_cdiv(units, 256)), dim3(256), 0, stream,
                     (const u32x4*)Wq, ldw / 16, (u32x4*)Wp, (int)(2 * I),
                     (int)ll_cdiv(I, tr / 2), units, (int)I, tr);
  LL_RETURN_LAUNCH();
}

namespace {

template <int MB, int NST, int TR, typename TO>
void launch_i8_gate_up(const int8_t* x, int64_t ldx, const int8_t* w, int64_t M, int64_t I,
                       int64_t K, unsigned tiles, const I8Epi& e, hipStream_t stream) {
  const size_t lds = (size_t)NST * (TR + 16 * MB) * 256;
  hipLaunchKernelGGL((gemm_dma_kernel<int8_t, MB, NST, true, 1, TR, TO>), dim3(tiles, 1),
                     dim3(256), lds, stream, x, ldx, w, K, (int)M, (int)(2 * I), (int)K,
                     (int)(K / 64), 0, nullptr, nullptr, 0, nullptr, e);
}

template <int MB, typename TO>
void launch_i8_gate_up_mb(const int8_t* x, int64_t ldx, const int8_t* w, int64_t M, int64_t I,
                          int64_t K, const I8Epi& e, hipStream_t stream) {
  const int tr = gate_up_tr(I);
  const unsigned tiles = (unsigned)ll_cdiv(I, tr / 2);
  if (tr == 128) launch_i8_gate_up<MB, 3, 128, TO>(x, ldx, w, M, I, K, tiles, e, stream);
  else if (tr == 96) launch_i8_gate_up<MB, 3, 96, TO>(x, ldx, w, M, I, K, tiles, e, stream);
  else if (tiles <= 256) launch_i8_gate_up<MB, 3, 64, TO>(x, ldx, w, M, I, K, tiles, e, stream);
  else launch_i8_gate_up<MB, 2, 64, TO>(x, ldx, w, M, I, K, tiles, e, stream);
}

}  // namespace

extern "C" int ll_gemm_i8_gate_up_silu_packed(const int8_t* Xq, int64_t ldx, const void* Wp,
                                              int64_t M, int64_t I, int64_t K, const float* s_tok,
                                              const void* s_ch, int s_ch_dtype, void* act,
                                              int64_t ld_act, int dtype, hipStream_t stream) {
  LL_CHECK_ARG(Xq && Wp && s_tok && s_ch && act, "ll_gemm_i8_gate_up_silu_packed: null pointer");
  LL_CHECK_ARG(M > 0 && M <= 64 && I > 0 && K > 0 && K % 256 == 0,
               "ll_gemm_i8_gate_up_silu_packed: needs 0 < M <= 64 and K %% 256 == 0");
  LL_CHECK_ARG(dtype == LL_BF16 || dtype == LL_F16, "ll_gemm_i8_gate_up_silu_packed: bf16/fp16 output");
  LL_CHECK_ARG(s_ch_dtype == LL_F32 || s_ch_dtype == LL_F16 || s_ch_dtype == LL_BF16,
               "ll_gemm_i8_gate_up_silu_packed: bad scale dtype %d", s_ch_dtype);
  LL_CHECK_ARG(ldx % 16 == 0 && (((uintptr_t)Xq | (uintptr_t)Wp) % 16) == 0,
               "ll_gemm_i8_gate_up_silu_packed: X rows must be 16 B aligned");
  const I8Epi e = {s_tok, s_ch, s_ch_dtype, act, ld_act};
  const int8_t* w = (const int8_t*)Wp;
  auto run = [&](auto tag) {
    typedef decltype(tag) TO;
    switch ((M + 15) / 16) {
      case 1: launch_i8_gate_up_mb<1, TO>(Xq, ldx, w, M, I, K, e, stream); break;
      case 2: launch_i8_gate_up_mb<2, TO>(Xq, ldx, w, M, I, K, e, stream); break;
      case 3: launch_i8_gate_up_mb<3, TO>(Xq, ldx, w, M, I, K, e, stream); break;
      default: launch_i8_gate_up_mb<4, TO>(Xq, ldx, w, M, I, K, e, stream); break;
    }
  };
  if (dtype == LL_BF16) run(__bf16{}); else run(_Float16{});
  LL_RETURN_LAUNCH();
}

extern "C" int ll_gemm_i8_splitk_count(int64_t M, int64_t N, int64_t K) {
  if (M > 64 || M <= 0 || K % 256 != 0) return 0;
  return plan_skinny(N, K, 1).splits;
}

extern "C" int ll_gemm_i8_splitk_packed(const int8_t* Xq, int64_t ldx, const void* Wp, int64_t M,
                                        int64_t N, int64_t K, int32_t* part, int64_t part_bytes,
                                        hipStream_t stream) {
  LL_CHECK_ARG(Xq && Wp && part, "ll_gemm_i8_splitk_packed: null pointer");
  LL_CHECK_ARG(M > 0 && M <= 64 && N > 0 && K > 0 && K % 256 == 0,
               "ll_gemm_i8_splitk_packed: needs 0 < M <= 64 and K %% 256 == 0");
  LL_CHECK_ARG(ldx % 16 == 0 && (((uintptr_t)Xq | (uintptr_t)Wp) % 16) == 0,
               "ll_gemm_i8_splitk_packed: X rows must be 16 B aligned");
  SkinnyPlan p = plan_skinny(N, K, 1);
  p.packed = true;
  p.rotate = 0;
  LL_CHECK_ARG(part_bytes >= (int64_t)p.splits * M * N * 4,
               "ll_gemm_i8_splitk_packed: partial buffer too small (need %lld bytes)",
               (long long)((int64_t)p.splits * M * N * 4));
  launch_skinny<int8_t>(p, Xq, ldx, (const int8_t*)Wp, K, nullptr, nullptr, 0, (float*)part,
                        (int)M, (int)N, (int)K, stream);
  LL_RETURN_LAUNCH();
}
