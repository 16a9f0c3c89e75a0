// Bandwidth-bound kernels of the Qwen2 token loop:
//   RMSNorm (+ fused residual add), RoPE (in place, drop-in form), the fused
//   RoPE + KV-cache scatter used by the model, SiLU_and_Mul, embedding gather,
//   and first-index argmax.
//
// Semantics follow the reference Triton kernels:
//   rmsnorm      litelang/kernel/develop_rmsnorm/rms_norm.py:20-59
//   rotary       litelang/kernel/develop_rope/rope.py:9-151
//   silu_and_mul litelang/kernel/develop_silu_and_mul/silu_and_mul.py:7-52
//   embedding    litelang/models/qwen2/layer/pre_layer.py:15-19
//   argmax       litelang/models/qwen2/layer/post_layer.py:75-77
#include "ll_common.h"

#include <string.h>

static thread_local char g_err[512];

void ll_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" const char* ll_last_error(void) { return g_err; }

extern "C" int ll_version(void) { return LL_ABI_VERSION; }

// ============================================================== RMSNorm
// An optional slot-table update done by a launch: req_to_tokens[rows[i],
// cols[i]] = slots[i] by thread 0 of grid row i (ll_assign_slots's update,
// folded into the decode step's first launch so that the step needs no
// launch of its own for it). r2t == nullptr: none.
struct LLSlotWrite {
  int32_t* r2t;
  int64_t stride;
  const int32_t* slots;
  const int32_t* rows;
  const int32_t* cols;
};

__device__ __forceinline__ void ll_slot_write(const LLSlotWrite& sw, int row) {
  if (sw.r2t != nullptr && threadIdx.x == 0)
    sw.r2t[(int64_t)sw.rows[row] * sw.stride + sw.cols[row]] = sw.slots[row];
}

// One workgroup per row. Pass 1 accumulates sum(x^2) in fp32, pass 2 scales.
// If `residual` is non-null the kernel first forms h = T(x + residual), stores
// it back into x (the reference's `hidden_states.add_()` at
// transformer_layer.py:69,76) and normalises h.
// With table: x[row] is first gathered from table[ids[row]] (the embedding;
// each thread re-reads only the elements it wrote); the id is clamped into
// [0, vocab) so the read stays inside the table.
template <typename T, int BLOCK>
__global__ __launch_bounds__(BLOCK) void rmsnorm_kernel(
    T* __restrict__ x, int64_t x_rs, const T* __restrict__ residual, int64_t r_rs,
    const T* __restrict__ gamma, T* __restrict__ out, int64_t o_rs, int N, float eps,
    const T* __restrict__ table, int64_t tab_rs, const void* ids, int ids64, int64_t vocab,
    uint32_t* __restrict__ bump, LLSlotWrite sw) {
  const int row = blockIdx.x;
  if (bump != nullptr && row == 0 && threadIdx.x == 0) *bump += 1u;
  ll_slot_write(sw, row);
  T* xr = x + (int64_t)row * x_rs;
  T* orow = out + (int64_t)row * o_rs;
  float ss = 0.f;
  if (table != nullptr) {
    int64_t id = ll_load_idx(ids, row, ids64);
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
    const T* src = table + id * tab_rs;
    for (int i = threadIdx.x; i < N; i += BLOCK) {
      const T h = src[i];
      xr[i] = h;
      float v = ll_to_f32(h);
      ss += v * v;
    }
  } else if (residual != nullptr) {
    const T* rr = residual + (int64_t)row * r_rs;
    for (int i = threadIdx.x; i < N; i += BLOCK) {
      T h = ll_from_f32<T>(ll_to_f32(xr[i]) + ll_to_f32(rr[i]));
      xr[i] = h;
      float v = ll_to_f32(h);
      ss += v * v;
    }
  } else {
    for (int i = threadIdx.x; i < N; i += BLOCK) {
      float v = ll_to_f32(xr[i]);
      ss += v * v;
    }
  }
  __shared__ float red[BLOCK / 64];
  ss = ll_wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < BLOCK / 64; ++w) tot += red[w];
  // reference: x / sqrt(sum(x^2)/N + eps) * gamma, all in fp32
  const float denom = sqrtf(tot / (float)N + eps);
  for (int i = threadIdx.x; i < N; i += BLOCK) {
    float v = ll_to_f32(xr[i]) / denom;
    orow[i] = ll_from_f32<T>(v * ll_to_f32(gamma[i]));
  }
}

// The same three forms for rows of N % 8 == 0 elements on 16-byte aligned
// rows (the model's hidden states): each thread holds up to C chunks of 8
// elements in registers (N <= 2048 C), so every element is read once with a
// 16-byte load and written once; the per-thread sum of squares runs over its
// chunks in order.
template <typename T, int C>
__global__ __launch_bounds__(256) void rmsnorm_vec8_kernel(
    T* __restrict__ x, int64_t x_rs, const T* __restrict__ residual, int64_t r_rs,
    const T* __restrict__ gamma, T* __restrict__ out, int64_t o_rs, int N, float eps,
    const T* __restrict__ table, int64_t tab_rs, const void* ids, int ids64, int64_t vocab,
    uint32_t* __restrict__ bump, LLSlotWrite sw) {
  typedef T V8 __attribute__((ext_vector_type(8)));
  const int row = blockIdx.x, nch = N / 8;
  if (bump != nullptr && row == 0 && threadIdx.x == 0) *bump += 1u;
  ll_slot_write(sw, row);
  T* xr = x + (int64_t)row * x_rs;
  const T* src = xr;
  if (table != nullptr) {
    int64_t id = ll_load_idx(ids, row, ids64);
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
    src = table + id * tab_rs;
  }
  V8 h[C];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int ch = threadIdx.x + 256 * c;
    if (ch < nch) {
      V8 v = *(const V8*)(src + 8 * ch);
      if (residual != nullptr) {
        const V8 r = *(const V8*)(residual + (int64_t)row * r_rs + 8 * ch);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = ll_from_f32<T>(ll_to_f32(v[e]) + ll_to_f32(r[e]));
      }
      if (table != nullptr || residual != nullptr) *(V8*)(xr + 8 * ch) = v;
      h[c] = v;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = ll_to_f32(v[e]);
        ss += f * f;
      }
    }
  }
  __shared__ float red[4];
  ss = ll_wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  // reference: x / sqrt(sum(x^2)/N + eps) * gamma, all in fp32
  const float denom = sqrtf(tot / (float)N + eps);
  T* orow = out + (int64_t)row * o_rs;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int ch = threadIdx.x + 256 * c;
    if (ch < nch) {
      const V8 g = *(const V8*)(gamma + 8 * ch);
      V8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = ll_from_f32<T>(ll_to_f32(h[c][e]) / denom * ll_to_f32(g[e]));
      *(V8*)(orow + 8 * ch) = o;
    }
  }
}

// Launch of the RMSNorm forms: the 16-byte kernel when N % 8 == 0, N <= 8192
// and every row is 16-byte aligned, the element-wise kernel otherwise.
template <typename T>
int launch_rmsnorm(T* x, int64_t x_rs, const T* residual, int64_t r_rs, const T* gamma, T* out,
                   int64_t o_rs, int64_t M, int64_t N, float eps, const T* table, int64_t tab_rs,
                   const void* ids, int ids64, int64_t vocab, hipStream_t stream,
                   uint32_t* bump = nullptr, const LLSlotWrite& sw = LLSlotWrite{}) {
  const auto al16 = [](const void* p, int64_t rs) {
    return ((uintptr_t)p % 16) == 0 && (rs * (int64_t)sizeof(T)) % 16 == 0;
  };
  const bool vec = N % 8 == 0 && N <= 8192 && al16(x, x_rs) && al16(gamma, 0) && al16(out, o_rs) &&
                   (residual == nullptr || al16(residual, r_rs)) &&
                   (table == nullptr || al16(table, tab_rs));
  if (vec) {
    const int C = (int)((N + 2047) / 2048);
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3((unsigned)M), dim3(256), 0, stream, x, x_rs, residual, r_rs,
                         gamma, out, o_rs, (int)N, eps, table, tab_rs, ids, ids64, vocab, bump, sw);
    };
    if (C == 1) go(rmsnorm_vec8_kernel<T, 1>);
    else if (C == 2) go(rmsnorm_vec8_kernel<T, 2>);
    else if (C == 3) go(rmsnorm_vec8_kernel<T, 3>);
    else go(rmsnorm_vec8_kernel<T, 4>);
  } else {
    hipLaunchKernelGGL((rmsnorm_kernel<T, 256>), dim3((unsigned)M), dim3(256), 0, stream, x, x_rs,
                       residual, r_rs, gamma, out, o_rs, (int)N, eps, table, tab_rs, ids, ids64,
                       vocab, bump, sw);
  }
  LL_RETURN_LAUNCH();
}

extern "C" int ll_rmsnorm(void* x, int64_t x_row_stride, const void* residual,
                          int64_t residual_row_stride, const void* gamma, void* out,
                          int64_t out_row_stride, int64_t M, int64_t N, float eps,
                          int dtype, hipStream_t stream) {
  LL_CHECK_ARG(x && gamma && out, "ll_rmsnorm: null pointer");
  LL_CHECK_ARG(M >= 0 && N > 0, "ll_rmsnorm: bad shape M=%lld N=%lld", (long long)M,
               (long long)N);
  if (M == 0) return LL_OK;
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    return launch_rmsnorm<T>((T*)x, x_row_stride, (const T*)residual, residual_row_stride,
                             (const T*)gamma, (T*)out, out_row_stride, M, N, eps, nullptr, 0,
                             nullptr, 0, 0, stream);
  });
}

// h[t] = table[ids[t]] and out[t] = rmsnorm(h[t]) * gamma in one launch: the
// results of ll_embedding followed by ll_rmsnorm, bit for bit. With a
// non-null `epoch`, the launch also adds 1 to that word (the decode step's
// epoch, which the step's fused launches read to tell their flags from the
// previous step's): the first launch of a decode step does it, so the step
// needs no launch of its own for it. The same launch can also do the step's
// slot-table update (sw).
namespace {
int embedding_rmsnorm_impl(const void* table, int64_t table_row_stride, int64_t vocab,
                           const void* ids, int ids_i64, void* h, int64_t h_row_stride,
                           const void* gamma, void* out, int64_t out_row_stride, int64_t ntok,
                           int64_t hidden, float eps, int dtype, uint32_t* epoch,
                           const LLSlotWrite& sw, hipStream_t stream) {
  LL_CHECK_ARG(table && ids && h && gamma && out, "ll_embedding_rmsnorm: null pointer");
  LL_CHECK_ARG(vocab > 0 && ntok >= 0 && hidden > 0, "ll_embedding_rmsnorm: bad shape");
  if (ntok == 0) return LL_OK;
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    return launch_rmsnorm<T>((T*)h, h_row_stride, nullptr, 0, (const T*)gamma, (T*)out,
                             out_row_stride, ntok, hidden, eps, (const T*)table, table_row_stride,
                             ids, ids_i64, vocab, stream, epoch, sw);
  });
}
}  // namespace

extern "C" int ll_embedding_rmsnorm(const void* table, int64_t table_row_stride, int64_t vocab,
                                    const void* ids, int ids_i64, void* h, int64_t h_row_stride,
                                    const void* gamma, void* out, int64_t out_row_stride,
                                    int64_t ntok, int64_t hidden, float eps, int dtype,
                                    hipStream_t stream) {
  return embedding_rmsnorm_impl(table, table_row_stride, vocab, ids, ids_i64, h, h_row_stride,
                                gamma, out, out_row_stride, ntok, hidden, eps, dtype, nullptr,
                                LLSlotWrite{}, stream);
}

extern "C" int ll_embedding_rmsnorm_epoch(const void* table, int64_t table_row_stride,
                                          int64_t vocab, const void* ids, int ids_i64, void* h,
                                          int64_t h_row_stride, const void* gamma, void* out,
                                          int64_t out_row_stride, int64_t ntok, int64_t hidden,
                                          float eps, int dtype, uint32_t* epoch,
                                          int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                                          const int32_t* slots, const int32_t* rows,
                                          const int32_t* cols, hipStream_t stream) {
  LL_CHECK_ARG(epoch != nullptr, "ll_embedding_rmsnorm_epoch: null epoch word");
  LL_CHECK_ARG(ntok > 0, "ll_embedding_rmsnorm_epoch: needs at least one token (the epoch "
                         "is advanced by the launch)");
  LL_CHECK_ARG(req_to_tokens == nullptr || (slots && rows && cols),
               "ll_embedding_rmsnorm_epoch: a slot-table update needs slots, rows and cols");
  const LLSlotWrite sw = {req_to_tokens, req_to_tokens_stride, slots, rows, cols};
  return embedding_rmsnorm_impl(table, table_row_stride, vocab, ids, ids_i64, h, h_row_stride,
                                gamma, out, out_row_stride, ntok, hidden, eps, dtype, epoch, sw,
                                stream);
}

// ============================================================== RoPE (drop-in)
// In place rotate-half on q [T, Hq, D] and k [T, Hk, D] (last dim contiguous,
// arbitrary token/head strides), with cos/sin already gathered per token
// [T, D/2]. One thread per (token, head, pair).
template <typename T, typename C>
__global__ void rope_kernel(T* __restrict__ q, int64_t q_st, int64_t q_sh, int Hq,
                            T* __restrict__ k, int64_t k_st, int64_t k_sh, int Hk,
                            const C* __restrict__ cs, int64_t c_st, const C* __restrict__ sn,
                            int64_t s_st, int64_t ntok, int half) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_tok = (int64_t)(Hq + Hk) * half;
  const int64_t t = gid / per_tok;
  if (t >= ntok) return;
  const int rem = (int)(gid - t * per_tok);
  const int h = rem / half;
  const int i = rem - h * half;
  T* base = (h < Hq) ? (q + t * q_st + (int64_t)h * q_sh) : (k + t * k_st + (int64_t)(h - Hq) * k_sh);
  const float c = ll_to_f32(cs[t * c_st + i]);
  const float s = ll_to_f32(sn[t * s_st + i]);
  const float x0 = ll_to_f32(base[i]);
  const float x1 = ll_to_f32(base[i + half]);
  ll_rope_pair(x0, x1, c, s, base[i], base[i + half]);
}

extern "C" int ll_rotary_emb(void* q, int64_t q_tok_stride, int64_t q_head_stride, int64_t q_heads,
                             void* k, int64_t k_tok_stride, int64_t k_head_stride, int64_t k_heads,
                             const void* cos, int64_t cos_tok_stride, const void* sin,
                             int64_t sin_tok_stride, int64_t ntok, int64_t head_dim, int dtype,
                             int cs_dtype, hipStream_t stream) {
  LL_CHECK_ARG(q && cos && sin, "ll_rotary_emb: null pointer");
  LL_CHECK_ARG(head_dim % 2 == 0 && head_dim > 0, "ll_rotary_emb: head_dim must be even");
  LL_CHECK_ARG(k_heads == 0 || k != nullptr, "ll_rotary_emb: null k");
  if (ntok == 0) return LL_OK;
  const int half = (int)(head_dim / 2);
  const int64_t total = ntok * (q_heads + k_heads) * half;
  const int block = 256;
  const unsigned grid = (unsigned)((total + block - 1) / block);
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    return LL_DISPATCH_DTYPE(cs_dtype, C, [&]() -> int {
      hipLaunchKernelGGL((rope_kernel<T, C>), dim3(grid), dim3(block), 0, stream, (T*)q,
                         q_tok_stride, q_head_stride, (int)q_heads, (T*)k, k_tok_stride,
                         k_head_stride, (int)k_heads, (const C*)cos, cos_tok_stride,
                         (const C*)sin, sin_tok_stride, ntok, half);
      LL_RETURN_LAUNCH();
    });
  });
}

// ============================================================== RoPE + KV scatter
// Model path for one layer. `qkv` is the projection output [T, (H + 2*KVH)*D]
// (q heads, then k heads, then v heads; row stride ld). For each token t:
//   q heads are rotated in place inside qkv;
//   k heads are rotated and written to pool[slot[t], 0:KVH, :];
//   v heads are copied to pool[slot[t], KVH:2*KVH, :].
// cos/sin come from the full table [max_len, D/2] indexed by position[t],
// replacing the index_select + gather + index_put sequence of
// transformer_layer.py:102-115,142-143.
template <typename T, typename C>
__global__ void rope_kv_scatter_kernel(T* __restrict__ qkv, int64_t ld, int H, int KVH, int D,
                                       const void* __restrict__ pos, int pos64,
                                       const C* __restrict__ cos_tab, const C* __restrict__ sin_tab,
                                       int64_t tab_stride, const int32_t* __restrict__ slots,
                                       T* __restrict__ pool, int64_t pool_slot_stride,
                                       int64_t pool_head_stride, int64_t ntok) {
  const int half = D / 2;
  const int64_t per_tok = (int64_t)(H + 2 * KVH) * half;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t t = gid / per_tok;
  if (t >= ntok) return;
  const int rem = (int)(gid - t * per_tok);
  const int h = rem / half;  // 0..H+2KVH-1
  const int i = rem - h * half;
  T* src = qkv + t * ld + (int64_t)h * D;
  if (h < H + KVH) {
    const int64_t p = ll_load_idx(pos, t, pos64);
    const float c = ll_to_f32(cos_tab[p * tab_stride + i]);
    const float s = ll_to_f32(sin_tab[p * tab_stride + i]);
    const float x0 = ll_to_f32(src[i]);
    const float x1 = ll_to_f32(src[i + half]);
    T y0, y1;
    ll_rope_pair(x0, x1, c, s, y0, y1);
    if (h < H) {
      src[i] = y0;
      src[i + half] = y1;
    } else {
      T* dst = pool + (int64_t)slots[t] * pool_slot_stride + (int64_t)(h - H) * pool_head_stride;
      dst[i] = y0;
      dst[i + half] = y1;
    }
  } else {
    T* dst = pool + (int64_t)slots[t] * pool_slot_stride + (int64_t)(h - H) * pool_head_stride;
    dst[i] = src[i];
    dst[i + half] = src[i + half];
  }
}

// The same, 4 rotation pairs per thread (8-byte loads and stores of the
// 16-bit types, head_dim % 8 == 0, 8-byte aligned rows): identical
// arithmetic per pair, a quarter of the threads and index math in 32 bits.
template <typename T, typename C>
__global__ __launch_bounds__(256) void rope_kv_scatter_vec4_kernel(
    T* __restrict__ qkv, int64_t ld, int H, int KVH, int D, const void* __restrict__ pos,
    int pos64, const C* __restrict__ cos_tab, const C* __restrict__ sin_tab, int64_t tab_stride,
    const int32_t* __restrict__ slots, T* __restrict__ pool, int64_t pool_slot_stride,
    int64_t pool_head_stride, int ntok) {
  typedef T V4 __attribute__((ext_vector_type(4)));
  const int half = D / 2, q4 = half / 4;
  const int per_tok = (H + 2 * KVH) * q4;
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const int t = gid / per_tok;
  if (t >= ntok) return;
  const int rem = gid - t * per_tok;
  const int h = rem / q4;
  const int i = (rem - h * q4) * 4;
  T* src = qkv + (int64_t)t * ld + (int64_t)h * D;
  const V4 a = *(const V4*)(src + i), b = *(const V4*)(src + i + half);
  V4 y0, y1;
  if (h < H + KVH) {
    const int64_t p = ll_load_idx(pos, t, pos64);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float cv = ll_to_f32(cos_tab[p * tab_stride + i + e]);
      const float sv = ll_to_f32(sin_tab[p * tab_stride + i + e]);
      T u, w;
      ll_rope_pair(ll_to_f32(a[e]), ll_to_f32(b[e]), cv, sv, u, w);
      y0[e] = u;
      y1[e] = w;
    }
  } else {
    y0 = a;
    y1 = b;
  }
  T* dst = h < H ? src
                 : pool + (int64_t)slots[t] * pool_slot_stride + (int64_t)(h - H) * pool_head_stride;
  *(V4*)(dst + i) = y0;
  *(V4*)(dst + i + half) = y1;
}

extern "C" int ll_rope_kv_scatter(void* qkv, int64_t qkv_row_stride, int64_t ntok, int64_t q_heads,
                                  int64_t kv_heads, int64_t head_dim, const void* positions,
                                  int positions_i64, const void* cos_table, const void* sin_table,
                                  int64_t table_row_stride, int cs_dtype, const int32_t* slots,
                                  void* pool_layer, int64_t pool_slot_stride,
                                  int64_t pool_head_stride, int dtype, hipStream_t stream) {
  LL_CHECK_ARG(qkv && positions && cos_table && sin_table && slots && pool_layer,
               "ll_rope_kv_scatter: null pointer");
  LL_CHECK_ARG(head_dim % 2 == 0, "ll_rope_kv_scatter: head_dim must be even");
  if (ntok == 0) return LL_OK;
  const int64_t total = ntok * (q_heads + 2 * kv_heads) * (head_dim / 2);
  const int block = 256;
  const unsigned grid = (unsigned)((total + block - 1) / block);
  const bool vec = (dtype == LL_BF16 || dtype == LL_F16) && head_dim % 8 == 0 &&
                   qkv_row_stride % 4 == 0 && pool_slot_stride % 4 == 0 &&
                   pool_head_stride % 4 == 0 && (((uintptr_t)qkv | (uintptr_t)pool_layer) % 8) == 0 &&
                   total / 4 < INT32_MAX;
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    return LL_DISPATCH_DTYPE(cs_dtype, C, [&]() -> int {
      if constexpr (sizeof(T) == 2) {
        if (vec) {
          hipLaunchKernelGGL((rope_kv_scatter_vec4_kernel<T, C>),
                             dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0, stream,
                             (T*)qkv, qkv_row_stride, (int)q_heads, (int)kv_heads,
                             (int)head_dim, positions, positions_i64, (const C*)cos_table,
                             (const C*)sin_table, table_row_stride, slots, (T*)pool_layer,
                             pool_slot_stride, pool_head_stride, (int)ntok);
          LL_RETURN_LAUNCH();
        }
      }
      hipLaunchKernelGGL((rope_kv_scatter_kernel<T, C>), dim3(grid), dim3(block), 0, stream,
                         (T*)qkv, qkv_row_stride, (int)q_heads, (int)kv_heads, (int)head_dim,
                         positions, positions_i64, (const C*)cos_table, (const C*)sin_table,
                         table_row_stride, slots, (T*)pool_layer, pool_slot_stride,
                         pool_head_stride, ntok);
      LL_RETURN_LAUNCH();
    });
  });
}

// ============================================================== KV store
// pool[slot[t], h, :] = src[t, h, :] for h < heads (plain scatter, no RoPE).
template <typename T>
__global__ void kv_store_kernel(const T* __restrict__ src, int64_t s_st, int64_t s_sh, int heads,
                                int D, const int32_t* __restrict__ slots, T* __restrict__ pool,
                                int64_t p_ss, int64_t p_sh, int64_t ntok) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_tok = (int64_t)heads * D;
  const int64_t t = gid / per_tok;
  if (t >= ntok) return;
  const int rem = (int)(gid - t * per_tok);
  const int h = rem / D, d = rem - h * D;
  pool[(int64_t)slots[t] * p_ss + (int64_t)h * p_sh + d] = src[t * s_st + (int64_t)h * s_sh + d];
}

extern "C" int ll_kv_store(const void* src, int64_t src_tok_stride, int64_t src_head_stride,
                           int64_t heads, int64_t head_dim, const int32_t* slots, void* pool,
                           int64_t pool_slot_stride, int64_t pool_head_stride, int64_t ntok,
                           int dtype, hipStream_t stream) {
  LL_CHECK_ARG(src && slots && pool, "ll_kv_store: null pointer");
  if (ntok == 0) return LL_OK;
  const int64_t total = ntok * heads * head_dim;
  const unsigned grid = (unsigned)((total + 255) / 256);
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    hipLaunchKernelGGL((kv_store_kernel<T>), dim3(grid), dim3(256), 0, stream, (const T*)src,
                       src_tok_stride, src_head_stride, (int)heads, (int)head_dim, slots, (T*)pool,
                       pool_slot_stride, pool_head_stride, ntok);
    LL_RETURN_LAUNCH();
  });
}

// ============================================================== SiLU_and_Mul
// out[m, n] = T( up * T(silu(gate)) ), gate = x[m, n], up = x[m, n + N].
// silu is evaluated in fp32 and rounded to the storage type before the
// multiply, as the reference does (silu_and_mul.py:43-50). `out` may alias x
// (the reference writes over the gate half in place).
template <typename T>
__global__ void silu_and_mul_kernel(const T* x, int64_t x_rs, T* out, int64_t o_rs, int64_t M,
                                    int N) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t m = gid / N;
  if (m >= M) return;
  const int n = (int)(gid - m * N);
  const float g = ll_to_f32(x[m * x_rs + n]);
  const float u = ll_to_f32(x[m * x_rs + n + N]);
  const T s = ll_from_f32<T>(ll_silu_f32(g));
  out[m * o_rs + n] = ll_from_f32<T>(u * ll_to_f32(s));
}

// Same, 8 elements (16 B) per thread for 16-bit types: one thread reads its
// gate and up chunks before writing, so in-place use stays safe.
template <typename T>
__global__ __launch_bounds__(256) void silu_and_mul_vec8_kernel(const T* x, int64_t x_rs, T* out,
                                                                int64_t o_rs, int64_t M, int N8) {
  typedef T V8 __attribute__((ext_vector_type(8)));
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t m = gid / N8;
  if (m >= M) return;
  const int n = (int)(gid - m * N8) * 8;
  const V8 g8 = *(const V8*)(x + m * x_rs + n);
  const V8 u8 = *(const V8*)(x + m * x_rs + n + (int64_t)N8 * 8);
  V8 o8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float g = ll_to_f32(g8[e]);
    const T s = ll_from_f32<T>(ll_silu_f32(g));
    o8[e] = ll_from_f32<T>(ll_to_f32(u8[e]) * ll_to_f32(s));
  }
  *(V8*)(out + m * o_rs + n) = o8;
}

extern "C" int ll_silu_and_mul(const void* x, int64_t x_row_stride, void* out,
                               int64_t out_row_stride, int64_t M, int64_t N, int dtype,
                               hipStream_t stream) {
  LL_CHECK_ARG(x && out, "ll_silu_and_mul: null pointer");
  if (M == 0 || N == 0) return LL_OK;
  const bool vec = (dtype == LL_BF16 || dtype == LL_F16) && N % 8 == 0 && x_row_stride % 8 == 0 &&
                   out_row_stride % 8 == 0 && (((uintptr_t)x | (uintptr_t)out) % 16) == 0;
  if (vec) {
    const unsigned grid = (unsigned)ll_cdiv(M * (N / 8), 256);
    if (dtype == LL_BF16)
      hipLaunchKernelGGL((silu_and_mul_vec8_kernel<__bf16>), dim3(grid), dim3(256), 0, stream,
                         (const __bf16*)x, x_row_stride, (__bf16*)out, out_row_stride, M, (int)(N / 8));
    else
      hipLaunchKernelGGL((silu_and_mul_vec8_kernel<_Float16>), dim3(grid), dim3(256), 0, stream,
                         (const _Float16*)x, x_row_stride, (_Float16*)out, out_row_stride, M,
                         (int)(N / 8));
    LL_RETURN_LAUNCH();
  }
  const int64_t total = M * N;
  const unsigned grid = (unsigned)((total + 255) / 256);
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    hipLaunchKernelGGL((silu_and_mul_kernel<T>), dim3(grid), dim3(256), 0, stream, (const T*)x,
                       x_row_stride, (T*)out, out_row_stride, M, (int)N);
    LL_RETURN_LAUNCH();
  });
}

// ============================================================== embedding
template <typename T>
__global__ void embedding_kernel(const T* __restrict__ table, int64_t tab_rs,
                                 const void* __restrict__ ids, int ids64, T* __restrict__ out,
                                 int64_t o_rs, int64_t ntok, int hidden, int64_t vocab) {
  const int64_t t = blockIdx.x;
  int64_t id = ll_load_idx(ids, t, ids64);
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // keep the read inside the table
  const T* src = table + id * tab_rs;
  T* dst = out + t * o_rs;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = src[i];
}

extern "C" int ll_embedding(const void* table, int64_t table_row_stride, int64_t vocab,
                            const void* ids, int ids_i64, void* out, int64_t out_row_stride,
                            int64_t ntok, int64_t hidden, int dtype, hipStream_t stream) {
  LL_CHECK_ARG(table && ids && out, "ll_embedding: null pointer");
  LL_CHECK_ARG(vocab > 0, "ll_embedding: empty table");
  if (ntok == 0) return LL_OK;
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    hipLaunchKernelGGL((embedding_kernel<T>), dim3((unsigned)ntok), dim3(256), 0, stream,
                       (const T*)table, table_row_stride, ids, ids_i64, (T*)out, out_row_stride,
                       ntok, (int)hidden, vocab);
    LL_RETURN_LAUNCH();
  });
}

// ============================================================== argmax
// out[m] = first index of the maximum of row m (torch.argmax tie rule), or
// -1 for every row when a status word is given and is nonzero (the decode
// step's fused launches set it when a flag wait gave up; -1 is no token id,
// so the host, which reads the tokens anyway, sees that the step is invalid).
// Pass 1: every workgroup reduces an 8192-wide chunk of a row to a
// (value, index) partial; pass 2 reduces the partials of each row. (Two
// launches: an in-launch last-workgroup merge would need a device-scope
// fence per workgroup, which flushes the XCD's whole L2 on gfx950.)
static const int kArgmaxChunk = 8192;   // elements per workgroup of pass 1
constexpr int kArgmaxChunkV = 8192;    // the same for the 16-byte-load pass

__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

__device__ __forceinline__ int64_t argmax_result(int bi, const uint32_t* status) {
  if (status != nullptr && *status != 0u) return -1;
  return (int64_t)(bi == 0x7fffffff ? 0 : bi);
}

__device__ __forceinline__ void argmax_block_reduce(float& v, int& i, float* sv, int* si) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    argmax_merge(v, i, ov, oi);
  }
  if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = v; si[threadIdx.x >> 6] = i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) argmax_merge(v, i, sv[w], si[w]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void argmax_partial_kernel(const T* __restrict__ x, int64_t x_rs,
                                                             int N, int chunk,
                                                             float* __restrict__ pval,
                                                             int* __restrict__ pidx,
                                                             int64_t* __restrict__ out,
                                                             const uint32_t* __restrict__ status) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int row = blockIdx.y, c = blockIdx.x, nchunk = gridDim.x;
  const T* xr = x + (int64_t)row * x_rs;
  const int beg = c * chunk, end = min(N, beg + chunk);
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = beg + threadIdx.x; i < end; i += 256) argmax_merge(best, bi, ll_to_f32(xr[i]), i);
  argmax_block_reduce(best, bi, sv, si);
  if (threadIdx.x == 0) {
    if (nchunk == 1) {
      out[row] = argmax_result(bi, status);
    } else {
      pval[row * nchunk + c] = best;
      pidx[row * nchunk + c] = bi;
    }
  }
}

// Pass 1 with 16-byte loads (VW = 16 / sizeof(T) elements each; rows 16 B
// aligned, N % VW == 0): every thread issues the loads of its whole share of
// the chunk before the first compare (clamped addresses, masked values),
// then merges them in index order, so the first-index rule holds as in the
// scalar pass.
template <typename T>
__global__ __launch_bounds__(256) void argmax_partial_vec_kernel(const T* __restrict__ x,
                                                                 int64_t x_rs, int N,
                                                                 float* __restrict__ pval,
                                                                 int* __restrict__ pidx,
                                                                 int64_t* __restrict__ out,
                                                                 const uint32_t* __restrict__ status) {
  constexpr int VW = 16 / (int)sizeof(T);
  typedef T VN __attribute__((ext_vector_type(VW)));
  constexpr int PER = kArgmaxChunkV / (256 * VW);  // 16-byte loads per thread
  __shared__ float sv[4];
  __shared__ int si[4];
  const int row = blockIdx.y, c = blockIdx.x, nchunk = gridDim.x;
  const T* xr = x + (int64_t)row * x_rs;
  const int beg = c * kArgmaxChunkV, end = min(N, beg + kArgmaxChunkV);
  VN v[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int p = beg + (q * 256 + (int)threadIdx.x) * VW;
    v[q] = *(const VN*)(xr + min(p, end - VW));
  }
  float best = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int p = beg + (q * 256 + (int)threadIdx.x) * VW;
    if (p < end) {
#pragma unroll
      for (int e = 0; e < VW; ++e) argmax_merge(best, bi, ll_to_f32(v[q][e]), p + e);
    }
  }
  argmax_block_reduce(best, bi, sv, si);
  if (threadIdx.x == 0) {
    if (nchunk == 1) {
      out[row] = argmax_result(bi, status);
    } else {
      pval[row * nchunk + c] = best;
      pidx[row * nchunk + c] = bi;
    }
  }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const float* __restrict__ pval,
                                                           const int* __restrict__ pidx,
                                                           int nchunk, int64_t* __restrict__ out,
                                                           const uint32_t* __restrict__ status) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int row = blockIdx.x;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < nchunk; i += 256)
    argmax_merge(best, bi, pval[row * nchunk + i], pidx[row * nchunk + i]);
  argmax_block_reduce(best, bi, sv, si);
  if (threadIdx.x == 0) out[row] = argmax_result(bi, status);
}


// The second pass on partials a producer wrote itself ([M][nparts] values
// and indices), for kernels that fold the first pass into their epilogue.
int ll_argmax_finish(const float* pval, const int* pidx, int64_t M, int64_t nparts, int64_t* out,
                     const uint32_t* status, hipStream_t stream) {
  LL_CHECK_ARG(pval && pidx && out && M > 0 && nparts > 0 && nparts < (1ll << 31),
               "ll_argmax_finish: bad arguments");
  hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)M), dim3(256), 0, stream, pval, pidx,
                     (int)nparts, out, status);
  LL_RETURN_LAUNCH();
}

extern "C" int64_t ll_argmax_workspace_size(int64_t M, int64_t N) {
  const int64_t nchunk = (N + kArgmaxChunk - 1) / kArgmaxChunk;
  return nchunk > 1 ? M * nchunk * 8 : 0;
}

namespace {
int argmax_impl(const void* x, int64_t x_row_stride, int64_t M, int64_t N, int64_t* out,
                void* workspace, int64_t workspace_bytes, int dtype, const uint32_t* status,
                hipStream_t stream) {
  LL_CHECK_ARG(x && out, "ll_argmax: null pointer");
  LL_CHECK_ARG(N > 0, "ll_argmax: empty rows");
  if (M == 0) return LL_OK;
  const int nchunk = ll_cdiv(N, kArgmaxChunk);
  float* pval = nullptr;
  int* pidx = nullptr;
  if (nchunk > 1) {
    LL_CHECK_ARG(workspace != nullptr && workspace_bytes >= ll_argmax_workspace_size(M, N),
                 "ll_argmax: workspace too small (need %lld bytes)",
                 (long long)ll_argmax_workspace_size(M, N));
    pval = (float*)workspace;
    pidx = (int*)(pval + M * nchunk);
  }
  const int vw = dtype == LL_F32 ? 4 : 8;  // elements per 16-byte load
  const bool vec = N % vw == 0 && x_row_stride % vw == 0 && ((uintptr_t)x % 16) == 0;
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    if (vec)
      hipLaunchKernelGGL((argmax_partial_vec_kernel<T>), dim3(nchunk, (unsigned)M), dim3(256), 0,
                         stream, (const T*)x, x_row_stride, (int)N, pval, pidx, out, status);
    else
      hipLaunchKernelGGL((argmax_partial_kernel<T>), dim3(nchunk, (unsigned)M), dim3(256), 0,
                         stream, (const T*)x, x_row_stride, (int)N, kArgmaxChunk, pval, pidx, out,
                         status);
    if (nchunk > 1)
      hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)M), dim3(256), 0, stream, pval, pidx,
                         nchunk, out, status);
    LL_RETURN_LAUNCH();
  });
}
}  // namespace

extern "C" int ll_argmax(const void* x, int64_t x_row_stride, int64_t M, int64_t N, int64_t* out,
                         void* workspace, int64_t workspace_bytes, int dtype, hipStream_t stream) {
  return argmax_impl(x, x_row_stride, M, N, out, workspace, workspace_bytes, dtype, nullptr,
                     stream);
}

extern "C" int ll_argmax_status(const void* x, int64_t x_row_stride, int64_t M, int64_t N,
                                int64_t* out, void* workspace, int64_t workspace_bytes, int dtype,
                                const uint32_t* status, hipStream_t stream) {
  LL_CHECK_ARG(status != nullptr, "ll_argmax_status: null status word");
  return argmax_impl(x, x_row_stride, M, N, out, workspace, workspace_bytes, dtype, status,
                     stream);
}

// ============================================================== slot table
// req_to_tokens[rows[i], cols[i]] = slots[i]: the table update of
// PageCache.alloc_token_idxs (litelang/models/cache.py:238-248) and
// PageCache.add_refs (cache.py:284-285), for host-computed (row, col) pairs.
__global__ void assign_slots_kernel(int32_t* __restrict__ r2t, int64_t r2t_stride,
                                    const int32_t* __restrict__ slots,
                                    const int32_t* __restrict__ rows,
                                    const int32_t* __restrict__ cols, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) r2t[(int64_t)rows[i] * r2t_stride + cols[i]] = slots[i];
}

extern "C" int ll_assign_slots(int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                               const int32_t* slots, const int32_t* rows, const int32_t* cols,
                               int64_t n, hipStream_t stream) {
  LL_CHECK_ARG(req_to_tokens && slots && rows && cols, "ll_assign_slots: null pointer");
  if (n == 0) return LL_OK;
  hipLaunchKernelGGL(assign_slots_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     req_to_tokens, req_to_tokens_stride, slots, rows, cols, n);
  LL_RETURN_LAUNCH();
}

// ============================================================== split-K consumers
// The decode-step projections leave fp32 partial sums part[s][m][n]
// (ll_gemm_splitk). The kernels below finish those sums in a fixed split
// order, store the projection output in the model dtype exactly as the
// unfused GEMM epilogue would (T(sum [+ bias])), and fuse the next op.

__device__ __forceinline__ float ll_sum_splits(const float* __restrict__ part, int splits,
                                               int64_t split_stride, int64_t idx) {
  float s = 0.f;
  for (int sp = 0; sp < splits; ++sp) s += part[sp * split_stride + idx];
  return s;
}

// h[m] = T(h[m] + T(sum_s part[s][m])); out[m] = rmsnorm(h[m]) * gamma.
// One workgroup per row, 4 consecutive columns per thread and pass (N % 4 == 0,
// N <= 4 * BLOCK * MAXP). The residual and gamma loads are unconditional (a
// clamped column) so they join the partials' memory round trip. With qout,
// the stored output row is also quantised per token (ll_quant_per_token's
// rule: s = max |out| / 127, 1 for a zero row) into qout / qscale.
template <typename T, int BLOCK, int MAXP>
__global__ __launch_bounds__(BLOCK) void add_rmsnorm_splitk_kernel(
    T* __restrict__ h, int64_t h_rs, const T* __restrict__ gamma, const void* __restrict__ part,
    int64_t part_sstride, int N, int splits_i32, LLPartials Pa, T* __restrict__ out, int64_t o_rs,
    int M, float eps, int8_t* __restrict__ qout, int64_t ldq, float* __restrict__ qscale) {
  // the first loads' fields (residual, gamma, partials, row length) are the
  // leading scalar arguments, which gfx950 preloads into SGPRs at dispatch,
  // so those loads do not wait for the load of the argument block; Pa
  // supplies the int32 partials' scales. splits_i32: splits | i32 << 16.
  LLPartials P = Pa;
  P.p = part;
  P.sstride = part_sstride;
  P.splits = splits_i32 & 0xffff;
  P.i32 = splits_i32 >> 16;
  constexpr int PER = 4;
  const int row = blockIdx.x;
  T* hr = h + (int64_t)row * h_rs;
  T hraw[MAXP][PER], graw[MAXP][PER];
#pragma unroll
  for (int ps = 0; ps < MAXP; ++ps) {
    const int c = min((ps * BLOCK + (int)threadIdx.x) * PER, N - PER);
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      hraw[ps][e] = hr[c + e];
      graw[ps][e] = gamma[c + e];
    }
  }
  float hv[MAXP][PER];
  float ss = 0.f;
#pragma unroll
  for (int ps = 0; ps < MAXP; ++ps) {
    const int c = (ps * BLOCK + threadIdx.x) * PER;
    if (c < N) {
      const f32x4 o = ll_partials_sum4(P, (int64_t)row * N + c, row, c);
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const T nh = ll_from_f32<T>(ll_to_f32(hraw[ps][e]) + ll_to_f32(ll_from_f32<T>(o[e])));
        hr[c + e] = nh;
        hv[ps][e] = ll_to_f32(nh);
        ss += hv[ps][e] * hv[ps][e];
      }
    }
  }
  __shared__ float red[BLOCK / 64];
  ss = ll_wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < BLOCK / 64; ++w) tot += red[w];
  const float denom = sqrtf(tot / (float)N + eps);
  T* orow = out + (int64_t)row * o_rs;
  float amax = 0.f;
#pragma unroll
  for (int ps = 0; ps < MAXP; ++ps) {
    const int c = (ps * BLOCK + threadIdx.x) * PER;
    if (c < N) {
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const T y = ll_from_f32<T>(hv[ps][e] / denom * ll_to_f32(graw[ps][e]));
        orow[c + e] = y;
        hv[ps][e] = ll_to_f32(y);
        amax = fmaxf(amax, fabsf(hv[ps][e]));
      }
    }
  }
  if (qout == nullptr) return;
  __shared__ float redm[BLOCK / 64];
  amax = ll_wave_max(amax);
  if ((threadIdx.x & 63) == 0) redm[threadIdx.x >> 6] = amax;
  __syncthreads();
  float m = 0.f;
#pragma unroll
  for (int w = 0; w < BLOCK / 64; ++w) m = fmaxf(m, redm[w]);
  float s = m / 127.f;
  if (!(s > 0.f)) s = 1.f;
  if (threadIdx.x == 0) qscale[row] = s;
  int8_t* qrow = qout + (int64_t)row * ldq;
#pragma unroll
  for (int ps = 0; ps < MAXP; ++ps) {
    const int c = (ps * BLOCK + threadIdx.x) * PER;
    if (c < N) {
#pragma unroll
      for (int e = 0; e < PER; ++e) qrow[c + e] = ll_quant1(hv[ps][e], s);
    }
  }
}

template <typename T, int MAXP>
void launch_add_rmsnorm_t(void* h, int64_t h_rs, const LLPartials& P, const void* gamma, void* out,
                          int64_t o_rs, int64_t M, int64_t N, float eps, int8_t* qout, int64_t ldq,
                          float* qscale, hipStream_t stream) {
  hipLaunchKernelGGL((add_rmsnorm_splitk_kernel<T, 512, MAXP>), dim3((unsigned)M), dim3(512), 0,
                     stream, (T*)h, h_rs, (const T*)gamma, P.p, P.sstride, (int)N,
                     P.splits | (P.i32 ? 1 << 16 : 0), P, (T*)out, o_rs, (int)M, eps, qout, ldq,
                     qscale);
}

int launch_add_rmsnorm(void* h, int64_t h_row_stride, const LLPartials& P, const void* gamma,
                       void* out, int64_t out_row_stride, int64_t M, int64_t N, float eps,
                       int dtype, int8_t* qout, int64_t ldq, float* qscale, hipStream_t stream) {
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    if (N <= 4 * 512)
      launch_add_rmsnorm_t<T, 1>(h, h_row_stride, P, gamma, out, out_row_stride, M, N, eps, qout,
                                 ldq, qscale, stream);
    else if (N <= 4 * 512 * 2)
      launch_add_rmsnorm_t<T, 2>(h, h_row_stride, P, gamma, out, out_row_stride, M, N, eps, qout,
                                 ldq, qscale, stream);
    else
      launch_add_rmsnorm_t<T, 4>(h, h_row_stride, P, gamma, out, out_row_stride, M, N, eps, qout,
                                 ldq, qscale, stream);
    LL_RETURN_LAUNCH();
  });
}

extern "C" int ll_add_rmsnorm_splitk(void* h, int64_t h_row_stride, const float* part, int splits,
                                     const void* gamma, void* out, int64_t out_row_stride,
                                     int64_t M, int64_t N, float eps, int dtype,
                                     hipStream_t stream) {
  LL_CHECK_ARG(h && part && gamma && out, "ll_add_rmsnorm_splitk: null pointer");
  LL_CHECK_ARG(splits >= 1 && splits < (1 << 16) && N > 0 && N % 4 == 0 && N <= 4 * 512 * 4,
               "ll_add_rmsnorm_splitk: N must be a multiple of 4 and <= 8192 (N=%lld), "
               "1 <= splits < 65536 (splits=%d)",
               (long long)N, splits);
  LL_CHECK_ARG(((uintptr_t)part) % 16 == 0, "ll_add_rmsnorm_splitk: partials must be 16 B aligned");
  if (M == 0) return LL_OK;
  return launch_add_rmsnorm(h, h_row_stride, ll_partials_f32(part, splits, M * N), gamma, out,
                            out_row_stride, M, N, eps, dtype, nullptr, 0, nullptr, stream);
}

extern "C" int ll_add_rmsnorm_splitk_i32(void* h, int64_t h_row_stride, const int32_t* part,
                                         int splits, const float* s_tok, const void* s_ch,
                                         int s_ch_dtype, const void* gamma, void* out,
                                         int64_t out_row_stride, int64_t M, int64_t N, float eps,
                                         int dtype, int8_t* q_out, int64_t ldq, float* q_scale,
                                         hipStream_t stream) {
  LL_CHECK_ARG(h && part && s_tok && s_ch && gamma && out, "ll_add_rmsnorm_splitk_i32: null pointer");
  LL_CHECK_ARG(splits >= 1 && splits < (1 << 16) && N > 0 && N % 4 == 0 && N <= 4 * 512 * 4,
               "ll_add_rmsnorm_splitk_i32: N must be a multiple of 4 and <= 8192 (N=%lld), "
               "1 <= splits < 65536 (splits=%d)",
               (long long)N, splits);
  LL_CHECK_ARG(((uintptr_t)part) % 16 == 0, "ll_add_rmsnorm_splitk_i32: partials must be 16 B aligned");
  LL_CHECK_ARG((q_out == nullptr) == (q_scale == nullptr) && (q_out == nullptr || ldq >= N),
               "ll_add_rmsnorm_splitk_i32: q_out and q_scale go together (ldq >= N)");
  LL_CHECK_ARG(s_ch_dtype == LL_F32 || s_ch_dtype == LL_F16 || s_ch_dtype == LL_BF16,
               "ll_add_rmsnorm_splitk_i32: bad scale dtype %d", s_ch_dtype);
  LL_CHECK_ARG(((uintptr_t)s_ch) % 4 == 0, "ll_add_rmsnorm_splitk_i32: s_ch must be 4 B aligned");
  if (M == 0) return LL_OK;
  LLPartials P = {part, splits, M * N, s_tok, s_ch, s_ch_dtype, 1};
  return launch_add_rmsnorm(h, h_row_stride, P, gamma, out, out_row_stride, M, N, eps, dtype,
                            q_out, ldq, q_scale, stream);
}

// out[m][n] = T(u * T(silu(g))), g = T(sum part[.][m][n]), u = T(sum part[.][m][N + n]);
// 4 consecutive columns per thread (N % 4 == 0).
template <typename T>
__global__ void silu_and_mul_splitk_kernel(LLPartials P, T* __restrict__ out, int64_t o_rs, int M,
                                           int N) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int q = N / 4;
  const int m = (int)(gid / q);
  if (m >= M) return;
  const int n = (int)(gid - (int64_t)m * q) * 4;
  const int64_t base = (int64_t)m * 2 * N;
  f32x4 g4, u4;
  ll_partials_sum4_pair(P, base + n, base + N + n, m, n, N + n, g4, u4);
  T* op = out + (int64_t)m * o_rs + n;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float g = ll_to_f32(ll_from_f32<T>(g4[e]));
    const float u = ll_to_f32(ll_from_f32<T>(u4[e]));
    const T sv = ll_from_f32<T>(ll_silu_f32(g));
    op[e] = ll_from_f32<T>(u * ll_to_f32(sv));
  }
}

int launch_silu_and_mul_splitk(const LLPartials& P, void* out, int64_t out_row_stride, int64_t M,
                               int64_t N, int dtype, hipStream_t stream) {
  const int64_t total = M * N / 4;
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    hipLaunchKernelGGL((silu_and_mul_splitk_kernel<T>), dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, stream, P, (T*)out, out_row_stride, (int)M, (int)N);
    LL_RETURN_LAUNCH();
  });
}

extern "C" int ll_silu_and_mul_splitk(const float* part, int splits, void* out,
                                      int64_t out_row_stride, int64_t M, int64_t N, int dtype,
                                      hipStream_t stream) {
  LL_CHECK_ARG(part && out, "ll_silu_and_mul_splitk: null pointer");
  LL_CHECK_ARG(N % 4 == 0 && ((uintptr_t)part) % 16 == 0,
               "ll_silu_and_mul_splitk: N must be a multiple of 4, partials 16 B aligned");
  if (M == 0 || N == 0) return LL_OK;
  return launch_silu_and_mul_splitk(ll_partials_f32(part, splits, M * 2 * N), out, out_row_stride,
                                    M, N, dtype, stream);
}

extern "C" int ll_silu_and_mul_splitk_i32(const int32_t* part, int splits, const float* s_tok,
                                          const void* s_ch, int s_ch_dtype, void* out,
                                          int64_t out_row_stride, int64_t M, int64_t N, int dtype,
                                          hipStream_t stream) {
  LL_CHECK_ARG(part && s_tok && s_ch && out, "ll_silu_and_mul_splitk_i32: null pointer");
  LL_CHECK_ARG(N % 4 == 0 && ((uintptr_t)part) % 16 == 0 && splits >= 1,
               "ll_silu_and_mul_splitk_i32: N must be a multiple of 4, partials 16 B aligned");
  LL_CHECK_ARG(s_ch_dtype == LL_F32 || s_ch_dtype == LL_F16 || s_ch_dtype == LL_BF16,
               "ll_silu_and_mul_splitk_i32: bad scale dtype %d", s_ch_dtype);
  LL_CHECK_ARG(((uintptr_t)s_ch) % 4 == 0, "ll_silu_and_mul_splitk_i32: s_ch must be 4 B aligned");
  if (M == 0 || N == 0) return LL_OK;
  LLPartials P = {part, splits, M * 2 * N, s_tok, s_ch, s_ch_dtype, 1};
  return launch_silu_and_mul_splitk(P, out, out_row_stride, M, N, dtype, stream);
}

// qkv = T(sum part + bias); q heads rotated -> q_out [T, H*D]; k rotated and
// v copied into pool_layer[slots[t]] (K heads then V heads). Each thread
// handles 4 consecutive rotation pairs (i..i+3, i+half..i+half+3); D % 8 == 0.
template <typename T, typename C>
__global__ void rope_kv_scatter_splitk_kernel(const float* __restrict__ part, int splits,
                                              const T* __restrict__ bias, T* __restrict__ q_out,
                                              int64_t q_rs, int H, int KVH, int D,
                                              const void* __restrict__ pos, int pos64,
                                              const C* __restrict__ cos_tab,
                                              const C* __restrict__ sin_tab, int64_t tab_stride,
                                              const int32_t* __restrict__ slots,
                                              T* __restrict__ pool, int64_t pool_slot_stride,
                                              int64_t pool_head_stride, int ntok) {
  const int half = D / 2;
  const int qd = half / 4;
  const int width = (H + 2 * KVH) * D;
  const int64_t per_tok = (int64_t)(H + 2 * KVH) * qd;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int t = (int)(gid / per_tok);
  if (t >= ntok) return;
  const int rem = (int)(gid - (int64_t)t * per_tok);
  const int h = rem / qd;
  const int i = (rem - h * qd) * 4;
  const int64_t sstride = (int64_t)ntok * width;
  const int c0 = h * D + i, c1 = c0 + half;
  f32x4 x0 = ll_sum_splits4(part, splits, sstride, (int64_t)t * width + c0);
  f32x4 x1 = ll_sum_splits4(part, splits, sstride, (int64_t)t * width + c1);
  if (bias != nullptr) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x0[e] += ll_to_f32(bias[c0 + e]);
      x1[e] += ll_to_f32(bias[c1 + e]);
    }
  }
  T* dst;
  if (h < H) dst = q_out + (int64_t)t * q_rs + (int64_t)h * D;
  else dst = pool + (int64_t)slots[t] * pool_slot_stride + (int64_t)(h - H) * pool_head_stride;
  if (h < H + KVH) {
    const int64_t p = ll_load_idx(pos, t, pos64);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c = ll_to_f32(cos_tab[p * tab_stride + i + e]);
      const float s = ll_to_f32(sin_tab[p * tab_stride + i + e]);
      const float a = ll_to_f32(ll_from_f32<T>(x0[e])), b = ll_to_f32(ll_from_f32<T>(x1[e]));
      ll_rope_pair(a, b, c, s, dst[i + e], dst[i + half + e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dst[i + e] = ll_from_f32<T>(x0[e]);
      dst[i + half + e] = ll_from_f32<T>(x1[e]);
    }
  }
}

extern "C" int ll_rope_kv_scatter_splitk(const float* part, int splits, const void* bias,
                                         void* q_out, int64_t q_row_stride, int64_t ntok,
                                         int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                         const void* positions, int positions_i64,
                                         const void* cos_table, const void* sin_table,
                                         int64_t table_row_stride, int cs_dtype,
                                         const int32_t* slots, void* pool_layer,
                                         int64_t pool_slot_stride, int64_t pool_head_stride,
                                         int dtype, hipStream_t stream) {
  LL_CHECK_ARG(part && q_out && positions && cos_table && sin_table && slots && pool_layer,
               "ll_rope_kv_scatter_splitk: null pointer");
  LL_CHECK_ARG(head_dim % 8 == 0 && ((uintptr_t)part) % 16 == 0,
               "ll_rope_kv_scatter_splitk: head_dim must be a multiple of 8, partials 16 B aligned");
  if (ntok == 0) return LL_OK;
  const int64_t total = ntok * (q_heads + 2 * kv_heads) * (head_dim / 8);
  const unsigned grid = (unsigned)((total + 255) / 256);
  return LL_DISPATCH_DTYPE(dtype, T, [&]() -> int {
    return LL_DISPATCH_DTYPE(cs_dtype, C, [&]() -> int {
      hipLaunchKernelGGL((rope_kv_scatter_splitk_kernel<T, C>), dim3(grid), dim3(256), 0, stream,
                         part, splits, (const T*)bias, (T*)q_out, q_row_stride, (int)q_heads,
                         (int)kv_heads, (int)head_dim, positions, positions_i64,
                         (const C*)cos_table, (const C*)sin_table, table_row_stride, slots,
                         (T*)pool_layer, pool_slot_stride, pool_head_stride, (int)ntok);
      LL_RETURN_LAUNCH();
    });
  });
}
