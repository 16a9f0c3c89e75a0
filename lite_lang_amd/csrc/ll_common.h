// Shared helpers for the lite_lang_amd HIP kernels (gfx950 / CDNA4 only).
//
// Storage types are the clang native `__bf16` and `_Float16`; every kernel
// computes in fp32 and rounds once on store (round-to-nearest-even).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Transposing LDS read (ds_read_b64_tr_b16, gfx950): within each group of 16
// lanes, lane i receives element i % 4 of the 8 bytes addressed by lane
// 4 e + i / 4, as its element e. Issued as inline asm: for the compiler's
// builtin of this instruction the wait insertion assumes that it may read
// what any LDS DMA still in flight writes, and waits for all of them
// (vmcnt(0)), which drains the copies of the tiles ahead of the one being
// read. The value is not there until ll_lds_wait_tie() has run on it.
__device__ __forceinline__ s16x4 ll_lds_read_tr16(const void* p) {
  s16x4 r;
  const uint32_t off =
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)(const char*)p;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(off) : "memory");
  return r;
}
// Wait for every LDS read of this wave (lgkmcnt(0)); the values read by
// ll_lds_read_tr16 pass through the wait as operands, so that no use of
// them can be scheduled before it.
template <int N> __device__ __forceinline__ void ll_lds_wait_tie(s16x4 (&v)[N]);
template <> __device__ __forceinline__ void ll_lds_wait_tie<4>(s16x4 (&v)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3])::"memory");
}
template <> __device__ __forceinline__ void ll_lds_wait_tie<8>(s16x4 (&v)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                 "+v"(v[6]), "+v"(v[7])::"memory");
}

#include "../../include/litelang_amd.h"

// short dtype names used inside the kernels
enum { LL_F32 = LL_DTYPE_F32, LL_F16 = LL_DTYPE_F16, LL_BF16 = LL_DTYPE_BF16 };

// Per-thread last-error text, returned by ll_last_error().
void ll_set_error(const char* fmt, ...);
// The host's spin setting for the decode step's bounded waits
// (ll_decode_sync_set_spin_limit: 0 = each wait's default, n > 0 = n polls,
// -n = test mode: the wait never sees its data and gives up after n polls).
int ll_decode_spin_setting();
// CUs of the current device, cached per device (gemm_tiles.hip): the
// persistent grids hold one workgroup per CU, each looping over its work.
int ll_device_cus(int* cus_out);

// Second pass of the first-index argmax over per-row partials [M][nparts]
// written by another kernel (elementwise.hip).
int ll_argmax_finish(const float* pval, const int* pidx, int64_t M, int64_t nparts, int64_t* out,
                     const uint32_t* status, hipStream_t stream);

#define LL_CHECK_ARG(cond, ...)                 \
  do {                                          \
    if (!(cond)) {                              \
      ll_set_error(__VA_ARGS__);                \
      return LL_ERR_ARG;                        \
    }                                           \
  } while (0)

#define LL_RETURN_LAUNCH()                                              \
  do {                                                                  \
    hipError_t _e = hipGetLastError();                                  \
    if (_e != hipSuccess) {                                             \
      ll_set_error("HIP launch failed: %s", hipGetErrorString(_e));     \
      return LL_ERR_HIP;                                                \
    }                                                                   \
    return LL_OK;                                                       \
  } while (0)

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float ll_to_f32(float x) { return x; }
__device__ __forceinline__ float ll_to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float ll_to_f32(__bf16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T ll_from_f32(float x);
template <>
__device__ __forceinline__ float ll_from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ _Float16 ll_from_f32<_Float16>(float x) { return (_Float16)x; }
template <>
__device__ __forceinline__ __bf16 ll_from_f32<__bf16>(float x) { return (__bf16)x; }

// silu(g) = g / (1 + exp(-g)) in fp32, the division done as a product with
// the reciprocal instruction (v_rcp_f32, 1 ulp) rather than the IEEE
// division sequence: the reference's Triton kernel divides with approximate
// fp32 division as well (litelang/kernel/develop_silu_and_mul/
// silu_and_mul.py:45). Every SiLU of the library goes through this function,
// so the fused GEMM epilogues and the standalone kernels round alike.
__device__ __forceinline__ float ll_silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// Index arrays arrive either as int32 or int64 (the reference builds them with
// torch.tensor(list) -> int64, and the slot table is int32).
__device__ __forceinline__ int64_t ll_load_idx(const void* p, int64_t i, int is64) {
  return is64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

// Up to U splits at once: every load is issued before the first addition (the
// split index is clamped so the loads need no branch; the surplus ones re-read
// the last split and are not added).
template <int U>
__device__ __forceinline__ f32x4 ll_sum_splits4_upto(const float* __restrict__ part, int splits,
                                                     int64_t split_stride, int64_t idx) {
  f32x4 v[U];
#pragma unroll
  for (int sp = 0; sp < U; ++sp)
    v[sp] = *(const f32x4*)(part + (int64_t)min(sp, splits - 1) * split_stride + idx);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < U; ++sp)
    if (sp < splits) acc += v[sp];
  return acc;
}

// Sum of 4 consecutive partial columns over all splits, added in split order
// 0, 1, 2, ... starting from +0. Up to 8 splits take one memory round trip;
// more splits go 4 loads at a time.
__device__ __forceinline__ f32x4 ll_sum_splits4(const float* __restrict__ part, int splits,
                                                int64_t split_stride, int64_t idx) {
  if (splits <= 4) return ll_sum_splits4_upto<4>(part, splits, split_stride, idx);
  if (splits <= 8) return ll_sum_splits4_upto<8>(part, splits, split_stride, idx);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int sp = 0;
  for (; sp + 4 <= splits; sp += 4) {
    const f32x4 a = *(const f32x4*)(part + (sp + 0) * split_stride + idx);
    const f32x4 b = *(const f32x4*)(part + (sp + 1) * split_stride + idx);
    const f32x4 c = *(const f32x4*)(part + (sp + 2) * split_stride + idx);
    const f32x4 d = *(const f32x4*)(part + (sp + 3) * split_stride + idx);
    acc += a;
    acc += b;
    acc += c;
    acc += d;
  }
  for (; sp < splits; ++sp) acc += *(const f32x4*)(part + sp * split_stride + idx);
  return acc;
}

// One int8 code: clamp(round_half_even(x / s), -128, 127) with IEEE division.
__device__ __forceinline__ int8_t ll_quant1(float x, float s) {
  float q = __builtin_rintf(x / s);
  q = fminf(fmaxf(q, -128.f), 127.f);
  return (int8_t)(int)q;
}

// int32 counterpart of ll_sum_splits4 (exact in any order).
__device__ __forceinline__ i32x4 ll_sum_splits4_i32(const int32_t* __restrict__ part, int splits,
                                                    int64_t split_stride, int64_t idx) {
  i32x4 acc = {0, 0, 0, 0};
  int sp = 0;
  if (splits <= 8) {
    i32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      v[u] = *(const i32x4*)(part + (int64_t)min(u, splits - 1) * split_stride + idx);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (u < splits) acc += v[u];
    return acc;
  }
  for (; sp < splits; ++sp) acc += *(const i32x4*)(part + sp * split_stride + idx);
  return acc;
}

// Split-K partial sums as the consumer kernels read them: fp32 partials (the
// bf16/fp16 GEMMs) or the W8A8 GEMM's int32 partials with their activation
// and channel scales, dequantised as fp32(sum) * s_tok[m] * fp32(s_ch[n]) --
// the arithmetic of ll_dequant_splitk, so a fused consumer equals dequant +
// the fp32 consumer bit for bit.
struct LLPartials {
  const void* p;        // const float* or const int32_t*
  int splits;
  int64_t sstride;      // elements between consecutive splits
  const float* s_tok;   // int32 partials: per-row activation scale [M]
  const void* s_ch;     // int32 partials: per-column weight scale [N]
  int s_ch_dtype;       // LL_F32 / LL_F16 / LL_BF16
  int i32;              // 1: int32 partials
};

__device__ __forceinline__ float ll_load_scale(const void* s, int dtype, int64_t i) {
  if (dtype == LL_F16) return (float)((const _Float16*)s)[i];
  if (dtype == LL_BF16) return (float)((const __bf16*)s)[i];
  return ((const float*)s)[i];
}

// A scale loaded as raw bits (fp32, or a zero-extended fp16 / bf16 code).
__device__ __forceinline__ float ll_scale_bits_to_f32(uint32_t bits, int dtype) {
  if (dtype == LL_F16) return (float)__builtin_bit_cast(_Float16, (unsigned short)bits);
  if (dtype == LL_BF16) return __builtin_bit_cast(float, bits << 16);
  return __builtin_bit_cast(float, bits);
}

// Columns col..col+3 of row m (idx = m * row_stride + col), summed over the splits.
__device__ __forceinline__ f32x4 ll_partials_sum4(const LLPartials& P, int64_t idx, int64_t m,
                                                  int64_t col) {
  if (!P.i32) return ll_sum_splits4((const float*)P.p, P.splits, P.sstride, idx);
  // the scales' raw bits are loaded ahead of the partials and converted after
  // the sum, so that all loads share one round trip (a conversion next to a
  // load under the dtype branch would wait for it there)
  // (16-bit scales as the two whole dwords holding them: col is a multiple of
  // 4 and s_ch 4-byte aligned; the halves are taken apart only at the end)
  const float st = P.s_tok[m];
  const uint32_t* sw = (const uint32_t*)P.s_ch;
  const bool f32 = P.s_ch_dtype == LL_F32;
  uint32_t sb[4];
  if (f32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) sb[e] = sw[col + e];
  } else {
    sb[0] = sw[col / 2];
    sb[1] = sw[col / 2 + 1];
    sb[2] = sb[3] = 0u;
  }
  const i32x4 acc = ll_sum_splits4_i32((const int32_t*)P.p, P.splits, P.sstride, idx);
  f32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t bits = f32 ? sb[e] : (sb[e >> 1] >> (16 * (e & 1))) & 0xffffu;
    o[e] = (float)acc[e] * st * ll_scale_bits_to_f32(bits, P.s_ch_dtype);
  }
  return o;
}

// Two column groups (idx0/col0 and idx1/col1) of ll_partials_sum4 with every
// load of both issued before either sum (one memory round trip for up to 8
// splits); each group is summed exactly as ll_partials_sum4 sums it.
template <int U>
__device__ __forceinline__ void ll_sum_splits4_pair_upto(const float* __restrict__ part, int splits,
                                                         int64_t ss, int64_t i0, int64_t i1,
                                                         f32x4& a0, f32x4& a1) {
  f32x4 v[U], w[U];
#pragma unroll
  for (int sp = 0; sp < U; ++sp) {
    const int64_t o = (int64_t)min(sp, splits - 1) * ss;
    v[sp] = *(const f32x4*)(part + o + i0);
    w[sp] = *(const f32x4*)(part + o + i1);
  }
  a0 = (f32x4){0.f, 0.f, 0.f, 0.f};
  a1 = a0;
#pragma unroll
  for (int sp = 0; sp < U; ++sp)
    if (sp < splits) {
      a0 += v[sp];
      a1 += w[sp];
    }
}

__device__ __forceinline__ void ll_partials_sum4_pair(const LLPartials& P, int64_t idx0,
                                                      int64_t idx1, int64_t m, int64_t col0,
                                                      int64_t col1, f32x4& o0, f32x4& o1) {
  if (P.splits > 8) {
    o0 = ll_partials_sum4(P, idx0, m, col0);
    o1 = ll_partials_sum4(P, idx1, m, col1);
    return;
  }
  if (!P.i32) {
    const float* part = (const float*)P.p;
    if (P.splits <= 4) ll_sum_splits4_pair_upto<4>(part, P.splits, P.sstride, idx0, idx1, o0, o1);
    else ll_sum_splits4_pair_upto<8>(part, P.splits, P.sstride, idx0, idx1, o0, o1);
    return;
  }
  const float st = P.s_tok[m];
  const uint32_t* sw = (const uint32_t*)P.s_ch;
  const bool f32 = P.s_ch_dtype == LL_F32;
  uint32_t sb0[4], sb1[4];
  if (f32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sb0[e] = sw[col0 + e];
      sb1[e] = sw[col1 + e];
    }
  } else {
    sb0[0] = sw[col0 / 2];
    sb0[1] = sw[col0 / 2 + 1];
    sb1[0] = sw[col1 / 2];
    sb1[1] = sw[col1 / 2 + 1];
    sb0[2] = sb0[3] = sb1[2] = sb1[3] = 0u;
  }
  const int32_t* part = (const int32_t*)P.p;
  i32x4 v[8], w[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int64_t o = (int64_t)min(u, P.splits - 1) * P.sstride;
    v[u] = *(const i32x4*)(part + o + idx0);
    w[u] = *(const i32x4*)(part + o + idx1);
  }
  i32x4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (u < P.splits) {
      a0 += v[u];
      a1 += w[u];
    }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t b0 = f32 ? sb0[e] : (sb0[e >> 1] >> (16 * (e & 1))) & 0xffffu;
    const uint32_t b1 = f32 ? sb1[e] : (sb1[e >> 1] >> (16 * (e & 1))) & 0xffffu;
    o0[e] = (float)a0[e] * st * ll_scale_bits_to_f32(b0, P.s_ch_dtype);
    o1[e] = (float)a1[e] * st * ll_scale_bits_to_f32(b1, P.s_ch_dtype);
  }
}

__host__ __device__ inline LLPartials ll_partials_f32(const float* p, int splits, int64_t sstride) {
  LLPartials P = {p, splits, sstride, nullptr, nullptr, 0, 0};
  return P;
}

// Rotate-half RoPE of one (x_i, x_{i+D/2}) pair, rounded to T. The fused
// multiply-adds are written out so every kernel rotating a pair rounds it the
// same way: y0 = fma(a, c, -(b*s)), y1 = fma(a, s, b*c).
// For fp16 the fp32 results are materialised before the conversion: otherwise
// the compiler may fuse fma + fp16 conversion into one mixed-precision
// instruction that rounds once, straight to fp16, where this sequence rounds
// to fp32 first (a one-ulp difference in rare cases, and between kernels).
// bf16 has no such fused instruction.
template <typename T>
__device__ __forceinline__ void ll_rope_pair(float a, float b, float c, float s, T& y0, T& y1) {
  float r0 = __builtin_fmaf(a, c, -(b * s));
  float r1 = __builtin_fmaf(a, s, b * c);
  if constexpr (sizeof(T) == 2 && !__is_same(T, __bf16)) asm volatile("" : "+v"(r0), "+v"(r1));
  y0 = ll_from_f32<T>(r0);
  y1 = ll_from_f32<T>(r1);
}

// ---------------------------------------------------------------- wave helpers
__device__ __forceinline__ float ll_wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float ll_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Dispatch a templated launcher on the runtime dtype code.
#define LL_DISPATCH_DTYPE(code, T, ...)                                  \
  [&]() -> int {                                                        \
    switch (code) {                                                     \
      case LL_F32: { typedef float T; return __VA_ARGS__(); }           \
      case LL_F16: { typedef _Float16 T; return __VA_ARGS__(); }        \
      case LL_BF16: { typedef __bf16 T; return __VA_ARGS__(); }         \
      default: ll_set_error("unsupported dtype code %d", (int)(code));   \
               return LL_ERR_UNSUPPORTED;                               \
    }                                                                   \
  }()

static inline int ll_cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
