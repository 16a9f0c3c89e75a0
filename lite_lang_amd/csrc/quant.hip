// W8A8 support: symmetric int8 quantisation of weights (per output channel)
// and activations (per token), and the dequantisation of int32 split-K
// partials into the fp32 partial format the fused consumer kernels read.
//
// Weight side follows quantize/smooth_quant/layer.py:5-16 on its float path:
//   s_o = T(max_i |w[o, i]| / 127)   (the scale is a tensor of the weight's dtype)
//   q   = clamp(round_half_even(fp32(w) / fp32(s_o)), -128, 127)
// Activation side is dynamic per token (the reference has no runtime
// activation quantisation; the north star fixes per-token absmax):
//   s_t = max_k |x[t, k]| / 127 in fp32 (1 when the row is all zeros)
//   q   = clamp(round_half_even(x / s_t), -128, 127)
// or static per tensor where a converted checkpoint carries a calibrated
// input scale (quant_scale of smooth_quant/layer.py:63-94): s_t = fp32(s_a).
// Dequantisation: y = fp32(sum of int32 partials) * s_t * fp32(s_o).
#include "ll_common.h"

namespace {

// Absolute maximum of a row, block-wide (blockDim.x == 256).
template <typename T>
__device__ float row_absmax(const T* __restrict__ row, int K, float* red) {
  float m = 0.f;
  for (int k = threadIdx.x; k < K; k += 256) m = fmaxf(m, fabsf(ll_to_f32(row[k])));
  m = ll_wave_max(m);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return m;
}

__device__ __forceinline__ int8_t quant1(float x, float s) { return ll_quant1(x, s); }

template <typename T>
__global__ __launch_bounds__(256) void quant_weight_kernel(const T* __restrict__ W, int64_t ldw,
                                                           int K, int8_t* __restrict__ Q,
                                                           int64_t ldq, T* __restrict__ scale) {
  __shared__ float red[4];
  const T* row = W + (int64_t)blockIdx.x * ldw;
  const float m = row_absmax(row, K, red);
  const T s_t = ll_from_f32<T>(m / 127.f);
  const float s = ll_to_f32(s_t);
  if (threadIdx.x == 0) scale[blockIdx.x] = s_t;
  int8_t* q = Q + (int64_t)blockIdx.x * ldq;
  for (int k = threadIdx.x; k < K; k += 256) q[k] = (s > 0.f) ? quant1(ll_to_f32(row[k]), s) : 0;
}

template <typename T> struct QVec8;
template <> struct QVec8<__bf16> { typedef bf16x8 type; };
template <> struct QVec8<_Float16> { typedef f16x8 type; };
typedef int8_t i8x8 __attribute__((ext_vector_type(8)));

// Vectorised row quantiser for bf16/fp16 rows with K % 8 == 0 (16 B aligned
// rows, 8 B aligned codes): each thread keeps VPT vectors of 8 elements in
// registers, so the row is read once. STATIC: scale = *s_static instead of
// the row absmax. Same arithmetic as the scalar kernels.
template <typename T, int VPT, bool STATIC>
__global__ __launch_bounds__(256) void quant_row_vec_kernel(const T* __restrict__ X, int64_t ldx,
                                                            int K, int8_t* __restrict__ Q,
                                                            int64_t ldq, float* __restrict__ scale,
                                                            const float* __restrict__ s_static) {
  typedef typename QVec8<T>::type V8;
  const T* row = X + (int64_t)blockIdx.x * ldx;
  // every load issued before the first use (clamped addresses; columns past
  // K are masked), one memory round trip for the row
  V8 v[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int k = (u * 256 + (int)threadIdx.x) * 8;
    v[u] = *(const V8*)(row + min(k, K - 8));
  }
  float m = 0.f;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int k = (u * 256 + (int)threadIdx.x) * 8;
    float mu = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) mu = fmaxf(mu, fabsf(ll_to_f32(v[u][e])));
    m = k < K ? fmaxf(m, mu) : m;
  }
  float s;
  if constexpr (STATIC) {
    s = *s_static;
  } else {
    __shared__ float red[4];
    m = ll_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    s = m / 127.f;
    if (!(s > 0.f)) s = 1.f;
  }
  if (threadIdx.x == 0) scale[blockIdx.x] = s;
  int8_t* q = Q + (int64_t)blockIdx.x * ldq;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int k = (u * 256 + (int)threadIdx.x) * 8;
    if (k < K) {
      i8x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = quant1(ll_to_f32(v[u][e]), s);
      *(i8x8*)(q + k) = o;
    }
  }
}

template <typename T, bool STATIC>
bool launch_quant_vec(const void* X, int64_t ldx, int64_t M, int64_t K, int8_t* Q, int64_t ldq,
                      float* scale, const float* s_static, hipStream_t stream) {
  if (K % 8 != 0 || ldx % 8 != 0 || ldq % 8 != 0 || ((uintptr_t)X % 16) != 0 ||
      ((uintptr_t)Q % 8) != 0 || K > 8 * 256 * 8)
    return false;
  const int vpt = (int)((K + 2047) / 2048);
  const dim3 grid((unsigned)M), block(256);
  if (vpt <= 1)
    hipLaunchKernelGGL((quant_row_vec_kernel<T, 1, STATIC>), grid, block, 0, stream, (const T*)X,
                       ldx, (int)K, Q, ldq, scale, s_static);
  else if (vpt <= 2)
    hipLaunchKernelGGL((quant_row_vec_kernel<T, 2, STATIC>), grid, block, 0, stream, (const T*)X,
                       ldx, (int)K, Q, ldq, scale, s_static);
  else if (vpt <= 4)
    hipLaunchKernelGGL((quant_row_vec_kernel<T, 4, STATIC>), grid, block, 0, stream, (const T*)X,
                       ldx, (int)K, Q, ldq, scale, s_static);
  else
    hipLaunchKernelGGL((quant_row_vec_kernel<T, 8, STATIC>), grid, block, 0, stream, (const T*)X,
                       ldx, (int)K, Q, ldq, scale, s_static);
  return true;
}

template <typename T>
__global__ __launch_bounds__(256) void quant_token_kernel(const T* __restrict__ X, int64_t ldx,
                                                          int K, int8_t* __restrict__ Q,
                                                          int64_t ldq, float* __restrict__ scale) {
  __shared__ float red[4];
  const T* row = X + (int64_t)blockIdx.x * ldx;
  const float m = row_absmax(row, K, red);
  float s = m / 127.f;
  if (!(s > 0.f)) s = 1.f;
  if (threadIdx.x == 0) scale[blockIdx.x] = s;
  int8_t* q = Q + (int64_t)blockIdx.x * ldq;
  for (int k = threadIdx.x; k < K; k += 256) q[k] = quant1(ll_to_f32(row[k]), s);
}

// Static per-tensor activation quantisation with a calibrated scale held in
// device memory (*scale > 0): q = clamp(rne(x / s)); s_tok[m] = s so that the
// dequantisation below applies unchanged.
template <typename T>
__global__ __launch_bounds__(256) void quant_static_kernel(const T* __restrict__ X, int64_t ldx,
                                                           int K, const float* __restrict__ scale,
                                                           int8_t* __restrict__ Q, int64_t ldq,
                                                           float* __restrict__ s_tok) {
  const float s = *scale;
  if (threadIdx.x == 0) s_tok[blockIdx.x] = s;
  const T* row = X + (int64_t)blockIdx.x * ldx;
  int8_t* q = Q + (int64_t)blockIdx.x * ldq;
  for (int k = threadIdx.x; k < K; k += 256) q[k] = quant1(ll_to_f32(row[k]), s);
}

// out[m][n] = fp32(sum_s part[s][m][n]) * s_tok[m] * fp32(s_ch[n]); 4 columns per thread
template <typename S>
__global__ __launch_bounds__(256) void dequant_splitk_kernel(const int32_t* __restrict__ part,
                                                             int splits, const float* __restrict__ s_tok,
                                                             const S* __restrict__ s_ch,
                                                             float* __restrict__ out, int M, int N) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int q = N / 4;
  const int m = (int)(gid / q);
  if (m >= M) return;
  const int n = (int)(gid - (int64_t)m * q) * 4;
  const int64_t stride = (int64_t)M * N;
  i32x4 acc = *(const i32x4*)(part + (int64_t)m * N + n);
  for (int sp = 1; sp < splits; ++sp) acc += *(const i32x4*)(part + sp * stride + (int64_t)m * N + n);
  const float st = s_tok[m];
  f32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = (float)acc[e] * st * ll_to_f32(s_ch[n + e]);
  *(f32x4*)(out + (int64_t)m * N + n) = o;
}

}  // namespace

extern "C" int ll_quant_weight_per_channel(const void* W, int64_t ldw, int64_t N, int64_t K,
                                           int dtype, int8_t* Q, int64_t ldq, void* scale,
                                           hipStream_t stream) {
  LL_CHECK_ARG(W && Q && scale, "ll_quant_weight_per_channel: null pointer");
  LL_CHECK_ARG(N >= 0 && K > 0 && ldw >= K && ldq >= K, "ll_quant_weight_per_channel: bad shape");
  if (N == 0) return LL_OK;
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    hipLaunchKernelGGL((quant_weight_kernel<T>), dim3((unsigned)N), dim3(256), 0, stream,
                       (const T*)W, ldw, (int)K, Q, ldq, (T*)scale);
    LL_RETURN_LAUNCH();
  });
}

extern "C" int ll_quant_per_token(const void* X, int64_t ldx, int64_t M, int64_t K, int dtype,
                                  int8_t* Q, int64_t ldq, float* scale, hipStream_t stream) {
  LL_CHECK_ARG(X && Q && scale, "ll_quant_per_token: null pointer");
  LL_CHECK_ARG(M >= 0 && K > 0 && ldx >= K && ldq >= K, "ll_quant_per_token: bad shape");
  if (M == 0) return LL_OK;
  if (dtype == LL_BF16 && launch_quant_vec<__bf16, false>(X, ldx, M, K, Q, ldq, scale, nullptr,
                                                          stream))
    LL_RETURN_LAUNCH();
  if (dtype == LL_F16 && launch_quant_vec<_Float16, false>(X, ldx, M, K, Q, ldq, scale, nullptr,
                                                           stream))
    LL_RETURN_LAUNCH();
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    hipLaunchKernelGGL((quant_token_kernel<T>), dim3((unsigned)M), dim3(256), 0, stream,
                       (const T*)X, ldx, (int)K, Q, ldq, scale);
    LL_RETURN_LAUNCH();
  });
}

extern "C" int ll_quant_static(const void* X, int64_t ldx, int64_t M, int64_t K, int dtype,
                               const float* scale, int8_t* Q, int64_t ldq, float* s_tok,
                               hipStream_t stream) {
  LL_CHECK_ARG(X && scale && Q && s_tok, "ll_quant_static: null pointer");
  LL_CHECK_ARG(M >= 0 && K > 0 && ldx >= K && ldq >= K, "ll_quant_static: bad shape");
  if (M == 0) return LL_OK;
  if (dtype == LL_BF16 && launch_quant_vec<__bf16, true>(X, ldx, M, K, Q, ldq, s_tok, scale,
                                                         stream))
    LL_RETURN_LAUNCH();
  if (dtype == LL_F16 && launch_quant_vec<_Float16, true>(X, ldx, M, K, Q, ldq, s_tok, scale,
                                                          stream))
    LL_RETURN_LAUNCH();
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    hipLaunchKernelGGL((quant_static_kernel<T>), dim3((unsigned)M), dim3(256), 0, stream,
                       (const T*)X, ldx, (int)K, scale, Q, ldq, s_tok);
    LL_RETURN_LAUNCH();
  });
}

extern "C" int ll_dequant_splitk(const int32_t* part, int splits, const float* s_tok,
                                 const void* s_ch, int s_ch_dtype, float* out, int64_t M,
                                 int64_t N, hipStream_t stream) {
  LL_CHECK_ARG(part && s_tok && s_ch && out, "ll_dequant_splitk: null pointer");
  LL_CHECK_ARG(splits >= 1 && M >= 0 && N > 0 && N % 4 == 0, "ll_dequant_splitk: needs N %% 4 == 0");
  if (M == 0) return LL_OK;
  const unsigned grid = (unsigned)ll_cdiv(M * (N / 4), 256);
  return LL_DISPATCH_DTYPE(s_ch_dtype, S, [&]() -> int {
    hipLaunchKernelGGL((dequant_splitk_kernel<S>), dim3(grid), dim3(256), 0, stream, part, splits,
                       s_tok, (const S*)s_ch, out, (int)M, (int)N);
    LL_RETURN_LAUNCH();
  });
}
