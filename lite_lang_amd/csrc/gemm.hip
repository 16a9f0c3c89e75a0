// Dense projections Y[M, N] = X[M, K] . W[N, K]^T (+ bias), gfx950.
//
// Replaces the cuBLAS products of the reference token loop
// (litelang/models/qwen2/layer/transformer_layer.py:80,82,95-109,193 and
// post_layer.py:50-52). W keeps the nn.Linear [out, in] layout so that both
// MFMA operands are 16-byte k-contiguous loads.
//
// Three kernels:
//   * skinny (M <= 64, the decode step): weight-streaming. A workgroup owns
//     16*WR output channels and a K range; its 4 waves interleave over the
//     32-wide k-steps with 4 steps in flight, multiply on MFMA
//     (v_mfma_f32_16x16x32) with the tokens as the 16-wide N side, and merge
//     in LDS. Narrow N is split over K across workgroups (fp32 partials,
//     reduced by a second kernel that also adds the bias);
//   * tiled (M > 64, prefill): 128x128x64 LDS tiles, 2x2 waves of 64x64,
//     register-staged prefetch of the next k tile;
//   * fp32: plain FMA tiles for the fp32 parity path.
#include "ll_common.h"

namespace {

template <typename T> struct Vec8;
template <> struct Vec8<__bf16> { typedef bf16x8 type; };
template <> struct Vec8<_Float16> { typedef f16x8 type; };

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <typename V8> __device__ __forceinline__ V8 zero8() {
  V8 z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = 0;
  return z;
}

// ---------------------------------------------------------------- skinny
constexpr int kSkWaves = 4;
constexpr int kSkUnroll = 4;

// grid.x = ceil(N / (16*WR)), grid.y = splits. Each split covers
// `ksteps_per_split` 32-wide k-steps.
template <typename T, int MB, int WR>
__global__ __launch_bounds__(kSkWaves * 64) void gemm_skinny_kernel(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ W, int64_t ldw,
    const T* __restrict__ bias, T* __restrict__ Y, int64_t ldy, float* __restrict__ part,
    int M, int N, int K, int ksteps_per_split) {
  typedef typename Vec8<T>::type V8;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, j = lane >> 4;
  const int row0 = blockIdx.x * (16 * WR);
  const int split = blockIdx.y;
  const int ksteps = (K + 31) / 32;
  const int kb = split * ksteps_per_split;
  const int ke = min(ksteps, kb + ksteps_per_split);

  const T* wrow[WR];
  bool wok[WR];
#pragma unroll
  for (int r = 0; r < WR; ++r) {
    const int row = row0 + 16 * r + n;
    wok[r] = row < N;
    wrow[r] = W + (int64_t)(wok[r] ? row : 0) * ldw + 8 * j;
  }
  const T* xrow[MB];
  bool xok[MB];
#pragma unroll
  for (int t = 0; t < MB; ++t) {
    const int tok = 16 * t + n;
    xok[t] = tok < M;
    xrow[t] = X + (int64_t)(xok[t] ? tok : 0) * ldx + 8 * j;
  }

  f32x4 acc[WR][MB];
#pragma unroll
  for (int r = 0; r < WR; ++r)
#pragma unroll
    for (int t = 0; t < MB; ++t) acc[r][t] = (f32x4){0.f, 0.f, 0.f, 0.f};

  for (int ks0 = kb + wave; ks0 < ke; ks0 += kSkWaves * kSkUnroll) {
    V8 wv[kSkUnroll][WR], xv[kSkUnroll][MB];
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u) {
      const int ks = ks0 + u * kSkWaves;
      const int k = ks * 32 + 8 * j;
      const bool kok = (ks < ke) && (k < K);
#pragma unroll
      for (int r = 0; r < WR; ++r)
        wv[u][r] = (kok && wok[r]) ? *(const V8*)(wrow[r] + ks * 32) : zero8<V8>();
#pragma unroll
      for (int t = 0; t < MB; ++t)
        xv[u][t] = (kok && xok[t]) ? *(const V8*)(xrow[t] + ks * 32) : zero8<V8>();
    }
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u)
#pragma unroll
      for (int r = 0; r < WR; ++r)
#pragma unroll
        for (int t = 0; t < MB; ++t) acc[r][t] = mfma16x16x32(wv[u][r], xv[u][t], acc[r][t]);
  }

  // acc[r][t][i] = Y[token 16t + n][channel row0 + 16r + 4j + i]
  __shared__ float red[kSkWaves][WR * 16][MB * 16 + 1];
#pragma unroll
  for (int r = 0; r < WR; ++r)
#pragma unroll
    for (int t = 0; t < MB; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][16 * r + 4 * j + i][16 * t + n] = acc[r][t][i];
  __syncthreads();
  for (int e = threadIdx.x; e < WR * 16 * MB * 16; e += kSkWaves * 64) {
    const int tok = e / (WR * 16);
    const int cr = e - tok * (WR * 16);
    const int ch = row0 + cr;
    if (tok >= M || ch >= N) continue;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kSkWaves; ++w) s += red[w][cr][tok];
    if (part != nullptr) {
      part[((int64_t)split * M + tok) * N + ch] = s;
    } else {
      if (bias != nullptr) s += ll_to_f32(bias[ch]);
      Y[(int64_t)tok * ldy + ch] = ll_from_f32<T>(s);
    }
  }
}

template <typename T>
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                     const T* __restrict__ bias, T* __restrict__ Y, int64_t ldy,
                                     int M, int N) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)M * N) return;
  const int tok = (int)(e / N), ch = (int)(e - (int64_t)tok * N);
  float s = 0.f;
  for (int sp = 0; sp < splits; ++sp) s += part[((int64_t)sp * M + tok) * N + ch];
  if (bias != nullptr) s += ll_to_f32(bias[ch]);
  Y[(int64_t)tok * ldy + ch] = ll_from_f32<T>(s);
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

struct SkinnyPlan {
  int wr;       // 16-row blocks per wave
  int splits;   // K splits across workgroups
  int ksps;     // k-steps per split
};

SkinnyPlan plan_skinny(int64_t N, int64_t K) {
  SkinnyPlan p;
  const int ksteps = (int)((K + 31) / 32);
  p.wr = (N >= 16 * 2 * 512) ? 2 : 1;  // wide N: 32 channels per workgroup
  const int64_t tiles = (N + 16 * p.wr - 1) / (16 * p.wr);
  // aim for >= 512 workgroups; each split keeps >= 4 k-steps per wave
  int splits = 1;
  while (tiles * splits < 512 && (ksteps / (splits * 2)) >= kSkWaves * 4) splits *= 2;
  p.splits = splits;
  p.ksps = (ksteps + splits - 1) / splits;
  p.splits = (ksteps + p.ksps - 1) / p.ksps;
  return p;
}

template <typename T, int MB>
int launch_skinny_mb(const SkinnyPlan& p, const T* X, int64_t ldx, const T* W, int64_t ldw,
                     const T* bias, T* Y, int64_t ldy, float* part, int M, int N, int K,
                     hipStream_t stream) {
  const dim3 grid((unsigned)ll_cdiv(N, 16 * p.wr), (unsigned)p.splits);
  if (p.wr == 2)
    hipLaunchKernelGGL((gemm_skinny_kernel<T, MB, 2>), grid, dim3(kSkWaves * 64), 0, stream, X,
                       ldx, W, ldw, bias, Y, ldy, part, M, N, K, p.ksps);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<T, MB, 1>), grid, dim3(kSkWaves * 64), 0, stream, X,
                       ldx, W, ldw, bias, Y, ldy, part, M, N, K, p.ksps);
  return 0;
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
    const int mb = (int)((M + 15) / 16);
    switch (mb) {
      case 1: launch_skinny_mb<T, 1>(p, X, ldx, W, ldw, bias, Y, ldy, part, (int)M, (int)N, (int)K, stream); break;
      case 2: launch_skinny_mb<T, 2>(p, X, ldx, W, ldw, bias, Y, ldy, part, (int)M, (int)N, (int)K, stream); break;
      case 3: launch_skinny_mb<T, 3>(p, X, ldx, W, ldw, bias, Y, ldy, part, (int)M, (int)N, (int)K, stream); break;
      default: launch_skinny_mb<T, 4>(p, X, ldx, W, ldw, bias, Y, ldy, part, (int)M, (int)N, (int)K, stream); break;
    }
    if (p.splits > 1) {
      const int64_t total = M * N;
      hipLaunchKernelGGL((splitk_reduce_kernel<T>), dim3((unsigned)((total + 255) / 256)), dim3(256),
                         0, stream, part, p.splits, bias, Y, ldy, (int)M, (int)N);
    }
    LL_RETURN_LAUNCH();
  }
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
